"""Decode benchmark: GPT-2 small greedy decode through the Vesta gfx950 kernel.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--batch 8] [--chunk 32]

One "step" is one greedy decode step of the whole batch: one pass of the
generated persistent kernel over the GPT-2 program (reference
``bench/g0_bench.py:166-180`` protocol: reset, untimed prefill one token per
launch, then timed back-to-back decode steps). Steps run ``--chunk`` per
cooperative launch (the kernel feeds each step's token back on the device).
Workload: GPT-2 small, random-init fp16 weights
N(0, 0.02) from seed 0, B=8 independent 128-token uniform-random prompts,
256 greedy tokens; the B=1 configuration is measured in the same
run and reported under "b1".

Prints ONE JSON line. ``roofline`` is for the one kernel: algorithmic bytes
per launch (weights once per step + the key/value rows of the context, the
reference's own accounting, ``vesta/gpt2.py:44-45,54-55``) over the average
launch duration measured with HIP events on the launch stream.
``cpu_baseline`` is this repository's CPU oracle (a NumPy restatement of the
reference interpreter) timed on this host on a bounded sample of the same
workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, 'vesta-gpu_amd'), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBPS = 8000.0
PROMPT, GEN = 128, 256


def step_bytes(m, n_ctx):
    """Reference accounting: weight bytes (wte counted once, one wpe row) plus
    keys and values of the context, per decode step."""
    return m.weight_bytes + m.kv_bytes(n_ctx)


def run_config(B, steps, warmup, chunk, seed=0):
    import torch
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts
    hf = RandomGPT2('small', seed)
    tmax = PROMPT + max(steps + warmup, GEN)
    tmax = min(1024, ((tmax + 63) // 64) * 64)
    m = VestaGPT2(hf, batch=B, tmax=tmax)
    prompts = torch.from_numpy(random_prompts(B, PROMPT, 50257, seed=1)).to('cuda', torch.int32)
    m.reset()
    m.prefill(prompts)          # one launch, one token per step (untimed)
    m.warm(warmup)              # untimed warm-up steps (same program, prefill kernel)
    torch.cuda.synchronize()
    plan = []
    left = steps
    while left > 0:
        n = min(chunk, left)
        plan.append(n)
        left -= n
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in plan]
    tokens = torch.zeros(steps * B, dtype=torch.int32, device='cuda')
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    off = 0
    for (a, b), n in zip(ev, plan):
        a.record()
        m.step(n, tokens[off * B:])
        b.record()
        off += n
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kern_ms = [a.elapsed_time(b) for a, b in ev]
    # algorithmic bytes of each launch: context grows by one per step
    pos0 = PROMPT + warmup
    per_launch_bytes, pos = [], pos0
    for n in plan:
        per_launch_bytes.append(sum(step_bytes(m, pos + k + 1) for k in range(n)))
        pos += n
    achieved = sum(per_launch_bytes) / (sum(kern_ms) / 1e3) / 1e9
    out = dict(B=B, steps=steps, tok_s=B * steps / elapsed, ms_per_step=elapsed / steps * 1e3,
               kernel_ms_per_launch=sum(kern_ms) / len(kern_ms), steps_per_launch=chunk,
               bytes_per_step_MB=step_bytes(m, pos0 + steps // 2) / 1e6, achieved_GBps=achieved,
               grid=m.k.grid, regs=m.k.attrs['regs'], barriers_per_step=m.low.barriers_per_launch + 1,
               weight_MB=m.weight_bytes / 1e6, tmax=tmax)
    del m
    torch.cuda.empty_cache()
    return out


def cpu_baseline(B, sample_steps):
    """The CPU oracle (NumPy restatement of the reference interpreter) on this
    host: ``sample_steps`` decode steps of each of B rows at the benchmark's
    mean context, one row at a time as the reference interpreter runs."""
    import numpy as np
    from oracle import decode
    from vesta.weights import RandomGPT2, stacked
    hf = RandomGPT2('small', 0)
    W = decode.oracle_weights(stacked(hf.numpy_state(), 12))
    text = open(os.path.join(ROOT, 'vesta-gpu_amd', 'vesta', 'programs', 'gpt2.vst')).read()
    rng = np.random.default_rng(2)
    t_mean = PROMPT + GEN // 2
    row = decode.Row(text, W, PROMPT + GEN)
    # a synthetic cache: CPU time does not depend on its values
    row.keys[:] = (rng.standard_normal(row.keys.shape) * 0.5).astype(np.float16)
    row.vals[:] = (rng.standard_normal(row.vals.shape) * 0.5).astype(np.float16)
    t0 = time.perf_counter()
    n = 0
    for b in range(B):
        for k in range(sample_steps):
            row.x, row.t = int(rng.integers(0, 50257)), t_mean + k
            row.step()
            n += 1
    dt = time.perf_counter() - t0
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    threads = os.environ.get('OPENBLAS_NUM_THREADS') or os.environ.get('OMP_NUM_THREADS') or str(cores)
    return dict(value=n / dt, unit='tok/s', cores=int(threads) if threads.isdigit() else cores, kind='port',
                sample=f'{sample_steps} decode steps x {B} rows of GPT-2 small at context {t_mean} '
                       f'(oracle/interp.py NumPy interpreter, one row at a time, {cores} host cores visible, '
                       f'BLAS threads {threads})')


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=GEN)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--batch', type=int, default=8)
    ap.add_argument('--chunk', type=int, default=32)
    ap.add_argument('--cpu-steps', type=int, default=2)
    ap.add_argument('--no-cpu', action='store_true')
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({'error': 'this build runs on one GPU: the decode step is one persistent kernel on one '
                                   'device; multi-GPU sharding is designed but not built (run with --gpus 1)'}))
        sys.exit(2)
    if args.steps + args.warmup + PROMPT > 1024:
        sys.exit('prompt + warmup + steps must stay within the 1024 learned positions')
    main_cfg = run_config(args.batch, args.steps, args.warmup, args.chunk)
    b1 = run_config(1, args.steps, args.warmup, args.chunk)
    peak = HBM_PEAK_GBPS
    line = {
        'metric': 'decode tok/s, GPT-2-small fp16 b1/b8; HBM GB/s as % of MI355X peak',
        'value': round(main_cfg['tok_s'], 1),
        'unit': 'tok/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(main_cfg['ms_per_step'], 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic: random-init GPT-2-small fp16 weights N(0,0.02) seed 0, uniform-random prompts',
        'config': {'workload': f'GPT-2 small greedy decode, B={args.batch}, {PROMPT}-token prompts, '
                               f'{args.steps} generated tokens (BASELINE.json configs[1])',
                   'batch': args.batch, 'prompt': PROMPT, 'storage': 'f16 weights and key/value cache, f32 math',
                   'steps_per_launch': args.chunk, 'grid': main_cfg['grid'],
                   'barriers_per_step': main_cfg['barriers_per_step']},
        'roofline': {'bound': 'hbm', 'achieved': round(main_cfg['achieved_GBps'], 1), 'peak': peak, 'unit': 'GB/s',
                     'frac': round(main_cfg['achieved_GBps'] / peak, 4), 'traffic': None,
                     'kernel': f'vesta_step_b{args.batch}', 'bytes_per_step_MB': round(main_cfg['bytes_per_step_MB'], 2),
                     'kernel_ms_per_launch': round(main_cfg['kernel_ms_per_launch'], 4)},
        'b1': {'tok_s': round(b1['tok_s'], 1), 'ms_per_step': round(b1['ms_per_step'], 4),
               'achieved_GBps': round(b1['achieved_GBps'], 1), 'frac': round(b1['achieved_GBps'] / peak, 4),
               'bytes_per_step_MB': round(b1['bytes_per_step_MB'], 2), 'grid': b1['grid'],
               'barriers_per_step': b1['barriers_per_step']},
    }
    if not args.no_cpu:
        line['cpu_baseline'] = cpu_baseline(args.batch, args.cpu_steps)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
