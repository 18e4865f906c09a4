"""Read the persistent kernel's own timing (reference ``timing=True``:
``vesta/lower.py:586-591``, ``vesta/gpt2.py:28,41``).

A model built with ``timing=True`` adds clock reads at every site boundary
of the generated kernel: each block sums, per site, the ticks spent since
the previous boundary, into ``Kernel.TS[site * grid + block]``. With
``timing='trace'`` only the launch's last step is traced: each block's
arrival and release time at every grid barrier, after the site table.
The clock is ``wall_clock64`` (100 MHz on MI355X).

    python -m vesta.profile sites|trace [--batch 8] [--steps 64] [--tmax 448]

prints a table of either for GPT-2 small at the benchmark's positions.
"""
from __future__ import annotations

import argparse
import time

import numpy as np

CLOCK_HZ = 100e6


def site_times(m, steps):
    """Run ``steps`` decode steps in one launch of a ``timing=True`` model.
    Returns (labels, us [sites, grid] per step, wall us per step)."""
    import torch
    k = m.k
    if k is None or m.low is None or m._timing is not True:
        raise ValueError('site times need the persistent kernel built with timing=True')
    k.TS.zero_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.step(steps)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e6
    ns = len(m.low.sites)
    ts = k.TS[:ns * k.grid].cpu().numpy().reshape(ns, k.grid).astype(np.float64)
    return list(m.low.sites), ts / steps / CLOCK_HZ * 1e6, wall


def barrier_labels(m):
    """The statement each grid barrier of one step comes before, in launch order."""
    src = [ln.split('// before ')[1] for ln in m.low.src.split('\n') if 'grid_arrive(bar);  // before ' in ln]
    loop = src.index('next l') + 1 if 'next l' in src else len(src)
    return src[:loop] * m.L + src[loop:]


def barrier_trace(m, steps=8):
    """Run ``steps`` steps in one launch of a ``timing='trace'`` model; for the
    last step, per barrier: (label, phase work before it as the slowest
    block's arrival after the previous release, arrival spread over blocks,
    release latency after the last arrival), all in us."""
    import torch
    from .lower import BTRACE
    k = m.k
    if k is None or m._timing != 'trace':
        raise ValueError("a barrier trace needs the persistent kernel built with timing='trace'")
    k.TS.zero_()
    m.step(steps)
    torch.cuda.synchronize()
    G = k.grid
    base = len(m.low.sites) * G
    tr = k.TS[base:base + 2 * BTRACE * G].cpu().numpy().reshape(BTRACE, 2, G).astype(np.int64)
    labels = barrier_labels(m)
    rows = []
    for i in range(BTRACE):
        arrive, release = tr[i, 0], tr[i, 1]
        if arrive.max() <= 0:
            break
        work = (arrive.max() - tr[i - 1, 1].min()) / CLOCK_HZ * 1e6 if i else None
        rows.append((labels[i] if i < len(labels) else f'#{i}', work,
                     (arrive.max() - arrive.min()) / CLOCK_HZ * 1e6,
                     (release.min() - arrive.max()) / CLOCK_HZ * 1e6))
    return rows


def _model(batch, tmax, timing, model='small', prompt=128, warm=118):
    import torch
    from .gpt2 import VestaGPT2
    from .weights import RandomGPT2, random_prompts
    m = VestaGPT2(RandomGPT2(model, 0), batch=batch, tmax=tmax, timing=timing, engine='persistent')
    m.reset()
    m.prefill(torch.from_numpy(random_prompts(batch, prompt, 50257, seed=1)).to('cuda', torch.int32))
    m.warm(warm)                       # by default to position 246: the benchmark's timed steps start there
    return m


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('what', choices=('sites', 'trace'))
    ap.add_argument('--batch', type=int, default=8)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--tmax', type=int, default=448)
    ap.add_argument('--model', default='small', choices=('small', 'medium', 'xl'))
    ap.add_argument('--prompt', type=int, default=128)
    ap.add_argument('--warm', type=int, default=118)
    a = ap.parse_args()
    if a.what == 'sites':
        m = _model(a.batch, a.tmax, True, a.model, a.prompt, a.warm)
        labels, us, wall = site_times(m, a.steps)
        print(f'GPT-2 {a.model} B={a.batch}, grid {m.k.grid}: wall {wall:.1f} us/step with timing marks; '
              f'block 0 sites sum to {us[:, 0].sum():.1f} us/step')
        agg = {}
        for lab, v in zip(labels, us[:, 0]):
            key = lab.split(':')[0]
            agg[key] = agg.get(key, 0.0) + v
        print('| site (block 0) | us per step |\n|---|---|')
        for key, v in sorted(agg.items(), key=lambda x: -x[1]):
            print(f'| {key} | {v:.1f} |')
        return
    m = _model(a.batch, a.tmax, 'trace', a.model, a.prompt, a.warm)
    rows = barrier_trace(m, a.steps)
    agg = {}
    for lab, work, spread, rel in rows:
        d = agg.setdefault(lab, [0, 0.0, 0.0, 0.0])
        d[0] += 1
        d[1] += work or 0.0
        d[2] += spread
        d[3] += rel
    print(f'GPT-2 {a.model} B={a.batch}, grid {m.k.grid}: {len(rows)} barriers in the last of {a.steps} steps '
          f'of one launch (positions from {a.prompt + a.warm})')
    print('| phase ends at the barrier before | barriers | work us (slowest block) | arrival spread us | '
          'release us |\n|---|---|---|---|---|')
    for lab, (n, w, s, r) in agg.items():
        print(f'| {lab} | {n} | {w:.1f} | {s:.1f} | {r:.1f} |')
    tw, tr = sum(d[1] for d in agg.values()), sum(d[3] for d in agg.values())
    print(f'| total | {len(rows)} | {tw:.1f} | | {tr:.1f} |')


if __name__ == '__main__':
    main()


# ------------------------------------------------------------------ device read bandwidth
READ_PROBE_SRC = r'''
typedef unsigned int vh_u32x4 __attribute__((ext_vector_type(4)));
// Streaming read of n16 16-byte words: every lane issues four nontemporal
// 16-byte loads per round (consecutive lanes, consecutive words), folding
// them into one XOR so no load is dead; one store if the fold hits a value
// the data never gives.
extern "C" __global__ __launch_bounds__(256) void vesta_read_probe(const vh_u32x4* __restrict__ p,
                                                                   unsigned long long n16,
                                                                   unsigned* __restrict__ out) {
  const unsigned long long stride = (unsigned long long)gridDim.x * 256ull;
  unsigned long long i = (unsigned long long)blockIdx.x * 256ull + threadIdx.x;
  vh_u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const vh_u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const vh_u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) out[0] = 1u;
}
'''


def stream_read_GBs(nbytes=512 << 20, blocks_per_cu=8, reps=20):
    """HBM read bandwidth of this device with the repository's own streaming
    read (``READ_PROBE_SRC``: 16-byte nontemporal loads, four in flight per
    lane), best of ``reps`` launches timed with HIP events on the launch
    stream; the buffer is ``nbytes`` of random data (well beyond the caches
    at the default 512 MB)."""
    import ctypes
    import torch
    from . import launch
    L = launch.lib()
    code = launch.compile_code(READ_PROBE_SRC)
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    launch.ok(L.vh_module_load(code, ctypes.byref(mod)), 'read probe load')
    try:
        launch.ok(L.vh_module_get_function(mod, b'vesta_read_probe', ctypes.byref(fn)), 'read probe function')
        n16 = nbytes // 16
        buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (n16 * 4,), dtype=torch.int32, device='cuda')
        out = torch.zeros(1, dtype=torch.int32, device='cuda')
        grid = launch.device_info()['cu_count'] * blocks_per_cu
        vals = [ctypes.c_void_p(buf.data_ptr()), ctypes.c_ulonglong(n16), ctypes.c_void_p(out.data_ptr())]
        args = (ctypes.c_void_p * 3)(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals])
        stream = torch.cuda.current_stream()
        best = None
        for r in range(reps + 3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            launch.ok(L.vh_launch(fn, grid, 256, 0, ctypes.c_void_p(stream.cuda_stream), args), 'read probe')
            e1.record(stream)
            e1.synchronize()
            if r >= 3:
                ms = e0.elapsed_time(e1)
                best = ms if best is None else min(best, ms)
        del buf, out
        return round(n16 * 16 / (best * 1e-3) / 1e9, 1)
    finally:
        launch.unload(mod)
