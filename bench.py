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
import csv
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, 'vesta-gpu_amd'), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBPS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0          # MI355X dense fp16 matrix-core peak
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'traffic.json')
PROMPT, GEN = 128, 256
MEAN_CTX = PROMPT + (GEN + 1) / 2       # mean context of configs[1]'s generated tokens: 256.5
BENCH_TMAX = 448                        # cache positions of the benchmarked kernels
REPEATS = 5                             # timed repeats; the median is reported (reference g0_bench.py:166-180)
CV_MAX = 0.05                           # repeats must agree within this coefficient of variation


def step_bytes(m, n_ctx):
    """Reference accounting: weight bytes (wte counted once, one wpe row) plus
    keys and values of the context, per decode step."""
    return m.weight_bytes + m.kv_bytes(n_ctx)


def step_flops(m, n_ctx):
    """Algorithmic FLOP of one decode step of B rows at context n_ctx: the
    four layer products and the tied head (2 per multiply-add), scores and
    weighted values over the context."""
    F = m.W['fcw'].shape[2]
    V = m.W['wte'].shape[0]
    return 2 * m.B * (m.L * (4 * m.D * m.D + 2 * m.D * F) + V * m.D) + 4 * m.B * m.L * n_ctx * m.D


def timed_start(steps, warmup):
    """Position of the first timed step. The timed steps are centred on the
    configuration's mean context (mean n_ctx of the timed steps = 256.5), after
    the prompt and the warm-up steps."""
    return max(PROMPT + warmup, int(round(MEAN_CTX - 0.5 - steps / 2)))


def bench_tmax(steps, warmup):
    need = timed_start(steps, warmup) + steps
    return BENCH_TMAX if need <= BENCH_TMAX else min(1024, -(-need // 64) * 64)


def make_model(B, tmax=BENCH_TMAX, seed=0):
    """The benchmarked model: GPT-2 small, random-init fp16 weights (seed 0),
    B rows, a ``tmax``-position cache. The parity tests build the kernels they
    check through here, so they check exactly the timed ones."""
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2
    return VestaGPT2(RandomGPT2('small', seed), batch=B, tmax=tmax)


def bench_prompts(B):
    from vesta.weights import random_prompts
    return random_prompts(B, PROMPT, 50257, seed=1)


def position(m, prompts, p0, warmup):
    """Reset, prefill the prompt (untimed, all positions together), decode up to
    position p0 - warmup (untimed), then ``warmup`` untimed warm-up steps: the
    next step runs at position p0."""
    m.reset()
    m.prefill(prompts)
    m.warm(p0 - PROMPT - warmup)
    m.warm(warmup)


def chunks(steps, chunk):
    plan, left = [], steps
    while left > 0:
        plan.append(min(chunk, left))
        left -= plan[-1]
    return plan


def _cv(xs):
    import statistics
    return statistics.pstdev(xs) / statistics.mean(xs) if len(xs) > 1 else 0.0


def run_config(B, steps, warmup, chunk, repeats=REPEATS, seed=0, single=True):
    """Decode throughput of GPT-2 small at B rows: ``repeats`` times (reset,
    prefill, positioning and warm-up steps, untimed) ``steps`` timed steps,
    ``chunk`` per launch (tokens fed back on the device); median and CV of
    the repeats. With ``single``, also the reference caller's protocol: one
    launch per step and a token copy after each (reference g0_bench.py:175-178),
    through the same program under its own kernel symbol so kernel profiles of
    the two legs stay apart."""
    import statistics
    import torch
    tmax = bench_tmax(steps, warmup)
    m = make_model(B, tmax, seed)
    prompts = torch.from_numpy(bench_prompts(B)).to('cuda', torch.int32)
    p0 = timed_start(steps, warmup)
    plan = chunks(steps, chunk)
    tokens = torch.zeros(steps * B, dtype=torch.int32, device='cuda')
    host, dev, first, same = [], [], None, True
    for _ in range(repeats):
        position(m, prompts, p0, warmup)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in plan]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        off = 0
        for (a, b), n in zip(ev, plan):
            a.record()
            m.step(n, tokens[off * B:])
            b.record()
            off += n
        torch.cuda.synchronize()
        host.append(time.perf_counter() - t0)
        dev.append(sum(a.elapsed_time(b) for a, b in ev) / 1e3)
        got = tokens.cpu()
        first = got if first is None else first
        same = same and bool(torch.equal(got, first))
    m.check()
    med_host, med_dev = statistics.median(host), statistics.median(dev)
    nbytes = sum(step_bytes(m, p0 + k + 1) for k in range(steps))
    nflop = sum(step_flops(m, p0 + k + 1) for k in range(steps))
    out = dict(B=B, steps=steps, tok_s=B * steps / med_host, ms_per_step=med_host / steps * 1e3,
               cv=_cv(host), device_ms_per_step=med_dev / steps * 1e3, device_cv=_cv(dev), repeats=repeats,
               repeats_identical_tokens=same, positions=[p0, p0 + steps - 1],
               mean_context=p0 + (steps + 1) / 2, kernel_ms_per_launch=med_dev * 1e3 / len(plan),
               steps_per_launch=steps / len(plan), launches=len(plan),
               bytes_per_step_MB=nbytes / steps / 1e6, achieved_GBps=nbytes / med_dev / 1e9,
               flop_per_step=nflop / steps, achieved_TFLOPs=nflop / med_dev / 1e12,
               algorithmic_bytes_per_launch=nbytes / len(plan), weight_MB=m.weight_bytes / 1e6, tmax=tmax,
               engine=m.engine)
    if m.k is not None:
        out.update(grid=m.k.grid, regs=m.k.attrs['regs'], kernel=m.low.name,
                   barriers_per_step=m.low.barriers_per_launch + ('feedback visible to the next step' in m.low.src),
                   src_sha=hashlib.sha256(m.low.src.encode()).hexdigest()[:16])
    else:
        out.update(grid=None, regs=None, kernel='layered', barriers_per_step=0, src_sha=None)
    if single:
        one = []
        step1 = m.variant(f'vesta_step1_b{B}') if m.k is not None else None
        for _ in range(repeats):
            position(m, prompts, p0, warmup)
            hist = []
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                if step1 is not None:
                    step1.launch(1)
                else:
                    m.step()
                hist.append(m.x.clone())
            torch.cuda.synchronize()
            one.append(time.perf_counter() - t0)
        m.check()
        med = statistics.median(one)
        out['one_launch_per_step'] = dict(tok_s=round(B * steps / med, 1), ms_per_step=round(med / steps * 1e3, 4),
                                          cv=round(_cv(one), 4),
                                          tokens_equal=bool(torch.equal(torch.stack(hist).view(-1).cpu(), first)))
    del m
    torch.cuda.empty_cache()
    return out


def device_bandwidth():
    """Copy and read bandwidth of this device (reference g0_bench.py:60-75:
    512 MB buffers, best of 20): the copy through PyTorch, the read with the
    repository's own streaming-read kernel (16-byte nontemporal loads, four
    in flight per lane; ``vesta.profile.stream_read_GBs``)."""
    import torch
    from vesta.profile import stream_read_GBs
    n = 256 * 1024 * 1024
    a = torch.empty(n, dtype=torch.float16, device='cuda').normal_()
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    ts = []
    for _ in range(20):
        t0 = time.perf_counter()
        b.copy_(a)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    out = {'copy_GBs': round(2 * n * 2 / min(ts) / 1e9, 1)}
    del a, b
    torch.cuda.empty_cache()
    out['read_GBs'] = stream_read_GBs(512 << 20)
    out['read_probe'] = '512 MB, own kernel: 16-byte nontemporal loads, best of 20 launches (HIP events)'
    return out


def measured_traffic(kernel, src_sha):
    """HBM bytes per launch of this exact kernel source as measured by two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; see --pmc-summary), or None
    when the committed measurement is for another source."""
    try:
        with open(TRAFFIC_FILE) as fh:
            table = json.load(fh)
    except (OSError, ValueError):
        return None
    rec = table.get(kernel)
    if not rec or rec.get('src_sha') != src_sha:
        return None
    return rec


def pmc_summary(fetch_csv, write_csv, bench_log, calib_mib):
    """Turn the counter CSVs of two profiled bench runs into HBM bytes per
    launch of each Vesta kernel. FETCH_SIZE and WRITE_SIZE (KiB per dispatch)
    are scaled so that the calibration copy of ``calib_mib`` MiB reads and
    writes exactly its size. Updates profiles/traffic.json and prints a
    markdown table."""
    want = calib_mib * 1024.0

    line = None
    for ln in open(bench_log):
        if ln.startswith('{') and '"metric"' in ln:
            line = json.loads(ln)
    if line is None:
        raise SystemExit(f'no bench JSON line in {bench_log}')
    cfgs = {line['roofline']['kernel']: line['roofline'], line['b1']['kernel']: line['b1']}

    def load(path):
        rows = list(csv.DictReader(open(path)))
        copies = [float(r['Counter_Value']) for r in rows if 'copyBuffer' in r['Kernel_Name']
                  or 'copy' in r['Kernel_Name'].lower()]
        calib = max(copies)
        per = {}
        for r in rows:
            if r['Kernel_Name'] in cfgs:           # the timed kernels only (not the one-launch-per-step leg's)
                per.setdefault(r['Kernel_Name'], []).append(float(r['Counter_Value']))
        return calib, per
    fc, fper = load(fetch_csv)
    wc, wper = load(write_csv)
    fscale, wscale = want / fc, want / wc
    table = {}
    if os.path.exists(TRAFFIC_FILE):
        table = json.load(open(TRAFFIC_FILE))
    print(f'| kernel | FETCH_SIZE KiB/launch | WRITE_SIZE KiB/launch | fetch bytes | write bytes | '
          f'algorithmic bytes | traffic / algorithmic |')
    print('|---|---|---|---|---|---|---|')
    for k in sorted(fper):
        f = sum(fper[k]) / len(fper[k])
        w = sum(wper.get(k, [0.0])) / max(1, len(wper.get(k, [])))
        fb, wb = f * 1024 * fscale, w * 1024 * wscale
        c = cfgs[k]
        alg = c['algorithmic_bytes_per_launch']
        table[k] = dict(src_sha=c['src_sha'], fetch_bytes=fb, write_bytes=wb, traffic=fb + wb,
                        algorithmic_bytes=alg, steps_per_launch=c['steps_per_launch'],
                        fetch_scale=fscale, write_scale=wscale,
                        run=f"steps {line.get('steps')}, warmup {line.get('warmup')}, positions "
                            f"{line.get('config', {}).get('positions')}")
        print(f'| {k} | {f:.0f} | {w:.0f} | {fb / 1e6:.1f} MB | {wb / 1e6:.1f} MB | {alg / 1e6:.1f} MB | '
              f'{(fb + wb) / alg:.3f} |')
    print(f'\nscale factors (calibration copy of {calib_mib} MiB): FETCH_SIZE x{fscale:.3f}, WRITE_SIZE x{wscale:.3f}')
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, 'w') as fh:
        json.dump(table, fh, indent=1, sort_keys=True)


def kernel_stats(db_path, top=12):
    """Markdown table of the kernel dispatches a ``rocprofv3 --kernel-trace``
    run recorded in its results database (rocpd SQLite): calls, mean and
    total duration per kernel, longest total first."""
    import sqlite3
    con = sqlite3.connect(db_path)
    rows = con.execute('select name, count(*), avg("end" - start), sum("end" - start) from kernels '
                       'group by name order by sum("end" - start) desc').fetchall()
    total = sum(r[3] for r in rows) or 1
    print('| kernel | calls | mean us | total ms | share |\n|---|---|---|---|---|')
    for name, n, mean, tot in rows[:top]:
        short = name if len(name) < 60 else name[:57] + '...'
        print(f'| {short} | {n} | {mean / 1e3:.3f} | {tot / 1e6:.3f} | {100 * tot / total:.1f}% |')


def calibration_copy(mib):
    """One device-to-device copy of ``mib`` MiB (reads and writes exactly that
    many bytes): the reference point for HBM traffic counters."""
    import torch
    n = mib << 20
    src = torch.ones(n // 4, dtype=torch.float32, device='cuda')
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


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


class TorchDecode:
    """Comparison arm, not the product: the same GPT-2 decode step written with
    PyTorch-ROCm operators (hipBLASLt GEMMs, fp16 storage and arithmetic), on
    the residues the Vesta kernel binds (reference arms ``bench/g0_bench.py:78-164``).

    Every step attends over the whole cache with positions past ``pos`` masked,
    so shapes are static and one step can be captured in a HIP graph. Keys are
    cached transposed (``[L, B, H, E, tmax]``) so both attention products are
    batched matrix products with contiguous right operands. ``step`` also feeds
    the chosen tokens back (``tok``, ``pos`` advance on the device)."""

    def __init__(self, W, n_head, batch, tmax):
        import torch
        self.W, self.B, self.H, self.tmax = W, batch, n_head, tmax
        self.L, self.D = W['qkvw'].shape[0], W['wte'].shape[1]
        self.E = self.D // n_head
        dt, dev = W['wte'].dtype, W['wte'].device
        self.kt = torch.zeros(self.L, batch, n_head, self.E, tmax, dtype=dt, device=dev)
        self.v = torch.zeros(self.L, batch, n_head, tmax, self.E, dtype=dt, device=dev)
        self.slots = torch.arange(tmax, device=dev)
        self.tok = torch.zeros(batch, dtype=torch.long, device=dev)
        self.pos = torch.zeros((), dtype=torch.long, device=dev)

    def reset(self):
        self.kt.zero_()
        self.v.zero_()
        self.pos.zero_()

    def step(self):
        import torch
        import torch.nn.functional as F
        W, B, H, E, D = self.W, self.B, self.H, self.E, self.D
        x = W['wte'].index_select(0, self.tok) + W['wpe'].index_select(0, self.pos.view(1))
        neg = torch.where(self.slots <= self.pos, 0.0, float('-inf')).to(x.dtype)
        at = self.pos.view(1)
        for l in range(self.L):
            h = F.layer_norm(x, (D,), W['ln1w'][l], W['ln1b'][l], 1e-5)
            q, k, v = torch.addmm(W['qkvb'][l], h, W['qkvw'][l]).view(B, 3, H, E).unbind(1)
            self.kt[l].index_copy_(3, at, k.unsqueeze(-1))
            self.v[l].index_copy_(2, at, v.unsqueeze(2))
            sc = torch.matmul(q.unsqueeze(2), self.kt[l]) * (E ** -0.5) + neg
            a = torch.matmul(torch.softmax(sc.float(), -1).to(x.dtype), self.v[l]).reshape(B, D)
            x = x + torch.addmm(W['ob'][l], a, W['ow'][l])
            h = F.layer_norm(x, (D,), W['ln2w'][l], W['ln2b'][l], 1e-5)
            h = F.gelu(torch.addmm(W['fcb'][l], h, W['fcw'][l]), approximate='tanh')
            x = x + torch.addmm(W['pb'][l], h, W['pw'][l])
        x = F.layer_norm(x, (D,), W['lnfw'], W['lnfb'], 1e-5)
        nxt = torch.matmul(x, W['wte'].t()).argmax(-1)
        self.tok.copy_(nxt)
        self.pos.add_(1)
        return nxt


def run_arm(name, B, steps, warmup, seed=0):
    """Tokens per second of one PyTorch arm on the benchmark workload
    (prompt fed one token per step untimed, ``warmup`` untimed steps, then
    ``steps`` timed steps), and its generated tokens [steps, B]."""
    import torch
    from vesta.gpt2 import gpt2_weights
    from vesta.weights import RandomGPT2, random_prompts
    W = {k: v.to('cuda', torch.float16).contiguous() for k, v in gpt2_weights(RandomGPT2('small', seed)).items()}
    tmax = min(1024, ((PROMPT + steps + warmup + 63) // 64) * 64)
    m = TorchDecode(W, 12, B, tmax)
    prompts = torch.from_numpy(random_prompts(B, PROMPT, 50257, seed=1)).to('cuda', torch.long)
    fn = m.step
    if name == 'torch_compile_graph':
        fn = torch.compile(m.step, fullgraph=True)
    graph = None
    if name in ('torch_graph', 'torch_compile_graph'):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()

    def one():
        if graph is not None:
            graph.replay()
        else:
            fn()
    m.reset()
    for i in range(PROMPT):
        m.tok.copy_(prompts[:, i])
        one()
    for _ in range(warmup):
        one()
    out = torch.zeros(steps, B, dtype=torch.long, device='cuda')
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        one()
        out[i].copy_(m.tok)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return B * steps / dt, out.cpu()


def arms_line(names, steps, warmup, batches=(1, 8)):
    """The PyTorch comparison arms beside the Vesta kernel on the same
    workload: tok/s per arm and batch, and whether each graph arm's tokens
    equal its eager run's (a HIP graph replay must reproduce eager results)."""
    import numpy as np
    res = {}
    for B in batches:
        vesta = run_config(B, steps, warmup, 32)
        res.setdefault('vesta', {})[f'b{B}'] = round(vesta['tok_s'], 1)
        eager_toks = None
        for name in names:
            tok_s, toks = run_arm(name, B, steps, warmup)
            rec = res.setdefault(name, {})
            rec[f'b{B}'] = round(tok_s, 1)
            if name == 'torch_eager':
                eager_toks = toks
            elif eager_toks is not None:
                rec[f'b{B}_tokens_equal_eager'] = bool(np.array_equal(toks.numpy(), eager_toks.numpy()))
    return {'metric': 'decode tok/s, GPT-2-small fp16, comparison arms on one MI355X', 'unit': 'tok/s',
            'steps': steps, 'warmup': warmup, 'prompt': PROMPT, 'arms': res,
            'note': 'torch arms: fp16 storage and arithmetic, whole-cache masked attention, one HIP graph per '
                    'step for the graph arms; vesta: the persistent kernel, 32 steps per launch'}


def prefill_line(shapes, reps=3):
    """Wall time of one prompt prefill per (B, P): all positions through each
    layer together (``mode='batched'``) against P decode steps in one launch
    (``mode='steps'``); each timed ``reps`` times (host clock around the call
    and a synchronize), the last one reported (the first pays compilation)."""
    import torch
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts
    out = {}
    for B, P in shapes:
        tmax = min(1024, max(384, ((P + 64 + 63) // 64) * 64))
        m = VestaGPT2(RandomGPT2('small', 0), batch=B, tmax=tmax)
        prompt = torch.from_numpy(random_prompts(B, P, 50257, seed=1)).to('cuda', torch.int32)
        rec = {}
        for mode in ('batched', 'steps'):
            for _ in range(reps):
                m.reset()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                m.prefill(prompt, mode=mode)
                torch.cuda.synchronize()
                rec[f'{mode}_ms'] = round((time.perf_counter() - t0) * 1e3, 3)
        rec['ratio'] = round(rec['steps_ms'] / rec['batched_ms'], 1)
        out[f'{B}x{P}'] = rec
        del m
        torch.cuda.empty_cache()
    return {'metric': 'prompt prefill wall time, GPT-2 small fp16, batched vs one decode step per position',
            'unit': 'ms', 'higher_is_better': False, 'shapes': out}


# BASELINE.json configurations beyond the benchmark line: (model, rows, prompt,
# generated tokens, cache positions)
CONFIGS = {3: ('small', 32, 768, 256, 1024), 4: ('medium', 8, 256, 256, 512), '4b1': ('medium', 1, 256, 256, 512),
           5: ('xl', 64, 128, 128, 256)}


def engines_line(shapes, steps=64, warmup=8, seed=0):
    """Both decode engines forced at each shape (model, rows, prompt, cache):
    ms per step of ``steps`` steps in one call after the batched prefill and
    ``warmup`` steps (the data behind ``gpt2.LAYERED_ROWS``)."""
    import torch
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts
    out = []
    for model, B, P, tmax in shapes:
        hf = RandomGPT2(model, seed)
        prompts = torch.from_numpy(random_prompts(B, P, 50257, seed=1)).to('cuda', torch.int32)
        row = dict(model=model, rows=B, prompt=P, tmax=tmax)
        for engine in ('persistent', 'layered'):
            try:
                m = VestaGPT2(hf, batch=B, tmax=tmax, engine=engine)
            except (RuntimeError, ValueError) as e:
                row[engine] = f'does not fit: {e}'[:120]
                continue
            m.reset()
            m.prefill(prompts)
            m.step(warmup)
            toks = torch.zeros(steps * B, dtype=torch.int32, device='cuda')
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            m.step(steps, toks)
            torch.cuda.synchronize()
            row[engine] = round((time.perf_counter() - t0) / steps * 1e3, 3)
            m.check()
            del m
            torch.cuda.empty_cache()
        out.append(row)
    return dict(metric='decode ms per step, both engines forced', unit='ms', rows=out)


def config_line(key, steps=None, warmup=8, chunk=32, seed=0, engine='auto'):
    """Greedy decode throughput of one of BASELINE.json's other configurations
    (random-init weights of that model, uniform-random prompts fed by the
    batched prefill, ``warmup`` untimed steps, then ``steps`` timed steps,
    ``chunk`` per launch), on the engine ``VestaGPT2(engine='auto')`` picks
    (from 11 rows of GPT-2 small, 9 of medium and at any row count of XL the
    layered engine, which measured faster there, runs each step as per-layer
    launches); the
    line says which engine ran, and ``engine`` forces one."""
    import torch
    from vesta.gpt2 import VestaGPT2
    from vesta.weights import RandomGPT2, random_prompts
    model, batch, prompt, gen, tmax = CONFIGS[key]
    steps = min(gen, tmax - prompt - warmup) if steps is None else steps
    if prompt + warmup + steps > tmax:
        sys.exit(f'prompt + warmup + steps must stay within the {tmax}-position cache of this configuration')
    m = VestaGPT2(RandomGPT2(model, seed), batch=batch, tmax=tmax, engine=engine)
    prompts = torch.from_numpy(random_prompts(batch, prompt, 50257, seed=1)).to('cuda', torch.int32)
    m.reset()
    m.prefill(prompts)
    m.warm(warmup)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    left = steps
    while left > 0:
        m.step(min(chunk, left))
        left -= chunk
    b.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    m.check()
    pos0 = prompt + warmup
    nbytes = sum(step_bytes(m, pos0 + k + 1) for k in range(steps))
    nflop = sum(step_flops(m, pos0 + k + 1) for k in range(steps))
    dev_s = a.elapsed_time(b) / 1e3
    return {'metric': f'decode tok/s, GPT-2-{model} fp16 b{batch} (BASELINE.json configs {key})',
            'value': round(batch * steps / elapsed, 1), 'unit': 'tok/s', 'ms_per_step': round(elapsed / steps * 1e3, 3),
            'steps': steps, 'warmup': warmup, 'prompt': prompt, 'tmax': tmax, 'engine': m.engine,
            'why': m.why_layered, 'grid': m.k.grid if m.k is not None else None,
            'hbm': {'achieved': round(nbytes / dev_s / 1e9, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
                    'frac': round(nbytes / dev_s / 1e9 / HBM_PEAK_GBPS, 4),
                    'bytes_per_step_MB': round(step_bytes(m, pos0 + steps // 2) / 1e6, 1)},
            'mfma': {'achieved': round(nflop / dev_s / 1e12, 2), 'peak': FP16_MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(nflop / dev_s / 1e12 / FP16_MFMA_PEAK_TFLOPS, 5),
                     'flop_per_step_G': round(nflop / steps / 1e9, 3)},
            'storage': STORAGE,
            'data': f'synthetic: random-init GPT-2-{model} fp16 weights N(0,0.02) seed {seed}, uniform-random prompts'}


def configs_summary():
    """BASELINE.json's other configurations in the default bench line (so
    the driver's own run measures them): each on the engine 'auto' picks,
    with the full step count of ``config_line``; for configurations 3 and 5,
    where 'auto' takes the layered engine, the persistent kernel's figure
    beside it."""
    import torch
    out = {}
    for key in (3, 4, '4b1', 5):
        try:
            c = config_line(key)
            row = {k: c[k] for k in ('value', 'unit', 'ms_per_step', 'steps', 'engine')}
            row['hbm_frac'] = c['hbm']['frac']
            row['mfma_frac'] = c['mfma']['frac']
            row['workload'] = c['metric'].split('(')[0].replace('decode tok/s, ', '').strip()
            if c['engine'] == 'layered':
                p = config_line(key, engine='persistent')
                row['persistent'] = {'ms_per_step': p['ms_per_step'], 'value': p['value'],
                                     'hbm_frac': p['hbm']['frac'], 'mfma_frac': p['mfma']['frac']}
        except Exception as e:           # one configuration failing must not take the benchmark line with it
            row = {'error': f'{type(e).__name__}: {e}'[:200]}
        out[str(key)] = row
        torch.cuda.empty_cache()
    return out


def xl_line(steps, warmup):
    """GPT-2 XL greedy decode at 64 rows."""
    return config_line(5, steps, warmup)


def roofline(cfg, peak):
    """The roofline object of one configuration's kernel: algorithmic bytes
    per launch over the launch duration (HIP events on the launch stream,
    median repeat), and the counter-measured HBM traffic per launch when
    profiles/traffic.json holds a measurement of this exact kernel source."""
    rec = measured_traffic(cfg['kernel'], cfg['src_sha']) if cfg['src_sha'] else None
    return {'bound': 'hbm', 'achieved': round(cfg['achieved_GBps'], 1), 'peak': peak, 'unit': 'GB/s',
            'frac': round(cfg['achieved_GBps'] / peak, 4),
            'traffic': round(rec['traffic']) if rec else None,
            'traffic_vs_algorithmic': round(rec['traffic'] / rec['algorithmic_bytes'], 3) if rec else None,
            'kernel': cfg['kernel'], 'src_sha': cfg['src_sha'], 'grid': cfg['grid'],
            'steps_per_launch': cfg['steps_per_launch'],
            'algorithmic_bytes_per_launch': round(cfg['algorithmic_bytes_per_launch']),
            'bytes_per_step_MB': round(cfg['bytes_per_step_MB'], 2),
            'kernel_ms_per_launch': round(cfg['kernel_ms_per_launch'], 4)}


def mfma_line(cfg):
    """Matrix-core utilisation: algorithmic FLOP over the timed device time
    against MI355X's dense fp16 peak (the products of a batched step run on
    the fp16 matrix cores; the activations go in as two fp16 halves, so the
    hardware does about twice the algorithmic product work)."""
    return {'achieved': round(cfg['achieved_TFLOPs'], 2), 'peak': FP16_MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
            'frac': round(cfg['achieved_TFLOPs'] / FP16_MFMA_PEAK_TFLOPS, 5),
            'flop_per_step_G': round(cfg['flop_per_step'] / 1e9, 3)}


def timing_line(cfg):
    return {'repeats': cfg['repeats'], 'cv': round(cfg['cv'], 4), 'device_cv': round(cfg['device_cv'], 4),
            'cv_ok': cfg['cv'] <= CV_MAX, 'repeats_identical_tokens': cfg['repeats_identical_tokens'],
            'device_ms_per_step': round(cfg['device_ms_per_step'], 4)}


STORAGE = ('f16 weights and key/value cache, f32 math; from 4 rows the products run on the fp16 matrix cores '
           'with each activation split into two fp16 halves (22 significant bits) and f32 accumulation')


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=GEN)
    ap.add_argument('--warmup', type=int, default=8)
    ap.add_argument('--batch', type=int, default=8)
    ap.add_argument('--chunk', type=int, default=32)
    ap.add_argument('--repeats', type=int, default=REPEATS)
    ap.add_argument('--cpu-steps', type=int, default=8)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--no-configs', action='store_true', help='leave configurations 3-5 out of the benchmark line')
    ap.add_argument('--pmc-summary', nargs=3, metavar=('FETCH_CSV', 'WRITE_CSV', 'BENCH_LOG'),
                    help='summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of '
                         '"bench.py --calibrate-copy N" into profiles/traffic.json and exit')
    ap.add_argument('--kernel-stats', metavar='DB',
                    help='print per-kernel dispatch statistics of a rocprofv3 --kernel-trace results database '
                         '(the *_results.db it writes) and exit')
    ap.add_argument('--calibrate-copy', type=int, default=0, metavar='MiB',
                    help='first run one plain device-to-device copy of this many MiB (a kernel of known '
                         'traffic, to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters)')
    ap.add_argument('--arms', default='', metavar='LIST',
                    help='instead of the benchmark line, time PyTorch comparison arms beside the Vesta kernel '
                         '(comma list of torch_eager, torch_graph, torch_compile_graph) at B=1 and B=8')
    ap.add_argument('--prefill', default='', metavar='BxP,...',
                    help='instead of the benchmark line, time prompt prefill (batched against one decode step '
                         'per position) for these shapes, e.g. 1x128,8x128')
    ap.add_argument('--xl', action='store_true',
                    help='instead of the benchmark line, measure GPT-2 XL decode at 64 rows (configs[4]); '
                         'give --steps 120 or fewer')
    ap.add_argument('--config', default='', metavar='KEY',
                    help='instead of the benchmark line, measure decode of another configuration: 3 (small, '
                         'B=32, 768-token prompts), 4 / 4b1 (medium, B=8 / B=1), 5 (XL, B=64)')
    ap.add_argument('--engine', default='auto', choices=('auto', 'persistent', 'layered'),
                    help='with --config: the decode engine (default: the one VestaGPT2 picks)')
    ap.add_argument('--engines', default='', metavar='MODEL:B:P:T,...',
                    help='instead of the benchmark line, time both decode engines forced at these shapes '
                         '(model, rows, prompt length, cache positions), e.g. small:16:128:448')
    args = ap.parse_args()
    if args.engines:
        shapes = [(m, int(b), int(p), int(t)) for m, b, p, t in (x.split(':') for x in args.engines.split(',') if x)]
        print(json.dumps(engines_line(shapes, args.steps if '--steps' in sys.argv else 64, args.warmup)), flush=True)
        return
    if args.config:
        key = int(args.config) if args.config.isdigit() else args.config
        if key not in CONFIGS:
            sys.exit(f'unknown configuration {args.config}')
        print(json.dumps(config_line(key, None if '--steps' not in sys.argv else args.steps, args.warmup,
                                     engine=args.engine)), flush=True)
        return
    if args.xl:
        print(json.dumps(xl_line(args.steps, args.warmup)), flush=True)
        return
    if args.prefill:
        shapes = [tuple(int(v) for v in x.split('x')) for x in args.prefill.split(',') if x]
        print(json.dumps(prefill_line(shapes)), flush=True)
        return
    if args.arms:
        names = [a for a in args.arms.split(',') if a]
        bad = set(names) - {'torch_eager', 'torch_graph', 'torch_compile_graph'}
        if bad:
            sys.exit(f'unknown arms: {sorted(bad)}')
        print(json.dumps(arms_line(names, args.steps, args.warmup)), flush=True)
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary, calib_mib=args.calibrate_copy or 1024)
        return
    if args.kernel_stats:
        kernel_stats(args.kernel_stats)
        return
    if args.gpus != 1:
        print(json.dumps({'error': 'this build runs on one GPU: the decode step is one persistent kernel on one '
                                   'device; multi-GPU sharding is designed but not built (run with --gpus 1)'}))
        sys.exit(2)
    if timed_start(args.steps, args.warmup) + args.steps > 1024:
        sys.exit('the timed steps must stay within the 1024 learned positions')
    if args.calibrate_copy > 0:
        calibration_copy(args.calibrate_copy)
    main_cfg = run_config(args.batch, args.steps, args.warmup, args.chunk, args.repeats)
    b1 = run_config(1, args.steps, args.warmup, args.chunk, args.repeats)
    peak = HBM_PEAK_GBPS
    p0, p1 = main_cfg['positions']
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
        'dtype': 'fp32 accumulate, 22-bit split activations from 4 rows',
        'data': 'synthetic: random-init GPT-2-small fp16 weights N(0,0.02) seed 0, uniform-random prompts',
        'config': {'workload': f'GPT-2 small greedy decode, B={args.batch}, {PROMPT}-token prompts (BASELINE.json '
                               f'configs[1]: 256 generated tokens, mean context {MEAN_CTX}); the {args.steps} '
                               f'timed steps run at positions {p0}..{p1} (mean context '
                               f'{main_cfg["mean_context"]}), after an untimed prefill and decode to position '
                               f'{p0}; median of {args.repeats} repeats',
                   'batch': args.batch, 'prompt': PROMPT, 'positions': [p0, p1], 'storage': STORAGE,
                   'engine': main_cfg['engine'], 'steps_per_launch': main_cfg['steps_per_launch'],
                   'barriers_per_step': main_cfg['barriers_per_step']},
        'timing': timing_line(main_cfg),
        'roofline': roofline(main_cfg, peak),
        'mfma': mfma_line(main_cfg),
        'one_launch_per_step': main_cfg.get('one_launch_per_step'),
        'b1': {'tok_s': round(b1['tok_s'], 1), 'ms_per_step': round(b1['ms_per_step'], 4),
               'barriers_per_step': b1['barriers_per_step'], 'timing': timing_line(b1),
               'one_launch_per_step': b1.get('one_launch_per_step'), **roofline(b1, peak)},
    }
    line['device_bandwidth'] = device_bandwidth()
    if not args.no_configs:
        line['configs'] = configs_summary()
    if not args.no_cpu:
        line['cpu_baseline'] = cpu_baseline(args.batch, args.cpu_steps)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
