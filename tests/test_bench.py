"""bench.py on the CPU: the one-GPU contract, and the HBM-traffic arithmetic
that turns two rocprofv3 --pmc runs into bytes per launch."""
import csv
import json
import os
import subprocess
import sys

import pytest

from conftest import REPO

sys.path.insert(0, REPO)
import bench  # noqa: E402


def _counters(path, rows):
    with open(path, 'w', newline='') as fh:
        w = csv.DictWriter(fh, fieldnames=['Kernel_Name', 'Counter_Name', 'Counter_Value'])
        w.writeheader()
        for name, value in rows:
            w.writerow({'Kernel_Name': name, 'Counter_Name': 'X', 'Counter_Value': value})


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, os.path.join(REPO, 'bench.py'), '--gpus', '2'], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2
    msg = json.loads(out.stdout.strip().splitlines()[-1])
    assert 'one GPU' in msg['error']


def test_pmc_summary_scales_counters_by_the_calibration_copy(tmp_path, monkeypatch, capsys):
    """A 1024 MiB copy that FETCH_SIZE reports as 524288 KiB and WRITE_SIZE as
    1048576 KiB gives scale factors 2 and 1; a kernel's bytes per launch are
    the mean counter over its dispatches times 1024 times the factor."""
    monkeypatch.setattr(bench, 'TRAFFIC_FILE', str(tmp_path / 'traffic.json'))
    fetch, write, log = tmp_path / 'f.csv', tmp_path / 'w.csv', tmp_path / 'bench.log'
    _counters(fetch, [('__amd_rocclr_copyBuffer', 524288.0), ('__amd_rocclr_copyBuffer', 3.0),
                      ('vesta_step_b8', 1000.0), ('vesta_step_b8', 3000.0), ('vesta_step_b1', 500.0),
                      ('vesta_step1_b8', 99999.0)])           # the one-launch-per-step leg: not averaged in
    _counters(write, [('__amd_rocclr_copyBuffer', 1048576.0), ('vesta_step_b8', 10.0), ('vesta_step_b1', 4.0)])
    line = {'metric': 'm', 'roofline': {'kernel': 'vesta_step_b8', 'src_sha': 'aa', 'steps_per_launch': 32,
                                        'algorithmic_bytes_per_launch': 8192000.0},
            'b1': {'kernel': 'vesta_step_b1', 'src_sha': 'bb', 'steps_per_launch': 32,
                   'algorithmic_bytes_per_launch': 1024000.0}}
    log.write_text('noise\n' + json.dumps(line) + '\n')
    bench.pmc_summary(str(fetch), str(write), str(log), 1024)
    table = json.load(open(bench.TRAFFIC_FILE))
    b8 = table['vesta_step_b8']
    assert b8['fetch_scale'] == pytest.approx(2.0) and b8['write_scale'] == pytest.approx(1.0)
    assert b8['fetch_bytes'] == pytest.approx(2000.0 * 1024 * 2)
    assert b8['write_bytes'] == pytest.approx(10.0 * 1024)
    assert b8['traffic'] == pytest.approx(2000.0 * 1024 * 2 + 10.0 * 1024)
    assert table['vesta_step_b1']['fetch_bytes'] == pytest.approx(500.0 * 1024 * 2)
    assert '| vesta_step_b8 |' in capsys.readouterr().out
    # the record is used only for the source it was measured on
    assert bench.measured_traffic('vesta_step_b8', 'aa')['traffic'] == b8['traffic']
    assert bench.measured_traffic('vesta_step_b8', 'cc') is None
    assert bench.measured_traffic('vesta_step_b4', 'aa') is None


def test_engines_mode_times_both_engines_at_each_shape(monkeypatch):
    """--engines parses model:rows:prompt:cache shapes and reports both
    engines' ms per step for each (the engine runs replaced by stand-ins)."""
    import types
    calls = []

    class FakeModel:
        def __init__(self, hf, batch, tmax, engine):
            calls.append((batch, tmax, engine))
            if engine == 'persistent' and batch > 16:
                raise RuntimeError('does not fit')

        def reset(self):
            pass

        def prefill(self, prompts):
            pass

        def step(self, n, tokens=None):
            pass

        def check(self):
            pass

    torch = pytest.importorskip('torch')
    fake_gpt2 = types.SimpleNamespace(VestaGPT2=FakeModel)
    monkeypatch.setitem(sys.modules, 'vesta.gpt2', fake_gpt2)
    monkeypatch.setattr(torch.cuda, 'synchronize', lambda: None)
    monkeypatch.setattr(torch.cuda, 'empty_cache', lambda: None)
    real_zeros, real_from_numpy = torch.zeros, torch.from_numpy
    monkeypatch.setattr(torch, 'zeros', lambda *a, **k: real_zeros(*a, **{x: y for x, y in k.items() if x != 'device'}))
    monkeypatch.setattr(torch.Tensor, 'to', lambda self, *a, **k: self)
    out = bench.engines_line([('small', 8, 4, 32), ('small', 32, 4, 64)], steps=2, warmup=1)
    rows = out['rows']
    assert [(r['rows'], r['tmax']) for r in rows] == [(8, 32), (32, 64)]
    assert isinstance(rows[0]['persistent'], float) and isinstance(rows[0]['layered'], float)
    assert rows[1]['persistent'].startswith('does not fit') and isinstance(rows[1]['layered'], float)
    assert calls == [(8, 32, 'persistent'), (8, 32, 'layered'), (32, 64, 'persistent'), (32, 64, 'layered')]
