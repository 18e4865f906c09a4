"""Phase emulator: run a lowered kernel's synchronisation skeleton under a
weak memory model and report every access that a missing grid barrier or
readiness flag would leave unordered.

The lowering decides where grid barriers go from its own static bookkeeping
(values written or read since the last barrier; reference
``vesta/lower.py:563-600`` keeps the same kind of table), and it removes
barriers three ways: readiness flags (a consumer waits only for the blocks
that made what it reads), local folds (a block folds only the values it made
itself, adding its partial sums into a fixed-point sum) and fixed-point sums
whose adds commute. This module checks those decisions independently, from
the events the code generation recorded in ``Lowering.trace`` in kernel
order:

    ('site', what, reads, writes)   a site begins; it reads / stores these values
    ('note', reads, writes)         more accesses of the current site
    ('store', z)                    the current site's writes of z are plain stores
                                    (a fixed-point sum's base), not atomic adds
    ('adds', z, reads)              a spread-out atomic add of z's base
    ('flags', what, values)         a new site that waits on readiness flags: the
                                    values its makers stored are visible to it
    ('clear', z, slot, ahead)       z cleared: before the arrival of the barrier
                                    opening prefetch slot ``slot``, or here (None)
    ('barrier', what, slot)         a grid barrier
    ('loop', var, n) / ('endloop', var)
    ('feedback', local, targets)    the step's feedback (block-local, or stores)

Memory model (what the kernel may rely on): a site's stores and adds become
visible to other sites only at the next grid barrier, or to a site that
waits on readiness flags for exactly those values. Within a phase (between
two barriers) the blocks run in any order, so a site may not read what
another site of the phase stores or adds (RAW), may not store or add what
another site of the phase read (WAR), and two sites may not both store one
value (WAW); atomic adds into one fixed-point sum from several sites commute
and are fine. Fixed-point sums kept in two buffers by layer parity resolve to
the buffer of the access: reads and plain adds the current layer's, the adds
into a layer loop's carry the next layer's, a clear the one it names. The
layer loop is unrolled over its extent and the step over ``steps``
iterations, the barrier between steps only where the kernel has one
(``Lowering.wrap_barrier``).

Accesses in the prefetch slots of barriers (weights, cache rows of earlier
positions) are not traced: the lowering issues early only loads of values
nobody writes or that were complete at the previous barrier.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class Race:
    kind: str            # 'RAW' | 'WAR' | 'WAW'
    value: str
    site: str            # the site making the second access
    other: str           # the site whose access it conflicts with
    step: int
    layer: int

    def __str__(self):
        return (f'{self.kind} on {self.value}: {self.site} vs {self.other} '
                f'(step {self.step}, layer counter {self.layer})')


@dataclass
class _Phase:
    stores: dict = field(default_factory=dict)    # value -> {site id: label}
    adds: dict = field(default_factory=dict)
    reads: dict = field(default_factory=dict)


def _expand(trace):
    """Nested list: events, with ('loop', var, n, body) for each loop."""
    out, stack = [], []
    cur = out
    for ev in trace:
        if ev[0] == 'loop':
            node = ['loop', ev[1], ev[2], []]
            cur.append(node)
            stack.append(cur)
            cur = node[3]
        elif ev[0] == 'endloop':
            cur = stack.pop()
        else:
            cur.append(ev)
    if stack:
        raise ValueError('unbalanced loop events in the trace')
    return out


class PhaseEmulator:
    def __init__(self, low):
        """``low``: the Lowering object (``_lower_once`` returns it)."""
        self.low = low
        self.parity = dict(getattr(low, 'fx_parity', {}))
        self.fx = set(getattr(low, 'fx', set()))
        self.races = []

    # ---------------------------------------------------------------- model
    def _buf(self, v, ahead=0, add=False):
        """The storage an access of v touches (parity buffers by layer)."""
        if v not in self.parity:
            return v
        kind = self.parity[v][3]
        if add and kind == 'carry':
            ahead = 1
        return f'{v}#{(self.layer + ahead) & 1}'

    def _race(self, kind, v, site, other):
        self.races.append(Race(kind, v, site, other, self.step, self.layer))

    def _read(self, v, sid, label, visible):
        b = self._buf(v)
        ph = self.ph
        for w in (ph.stores.get(b, {}), ph.adds.get(b, {})):
            for osid, olabel in w.items():
                if osid != sid and v not in visible:
                    self._race('RAW', b, label, olabel)
        ph.reads.setdefault(b, {})[sid] = label

    def _write(self, v, sid, label, mode, ahead=0):
        b = self._buf(v, ahead, add=(mode == 'add'))
        ph = self.ph
        for osid, olabel in ph.reads.get(b, {}).items():
            if osid != sid:
                self._race('WAR', b, label, olabel)
        for osid, olabel in ph.stores.get(b, {}).items():
            if osid != sid:
                self._race('WAW', b, label, olabel)
        if mode != 'add':
            for osid, olabel in ph.adds.get(b, {}).items():
                if osid != sid:
                    self._race('WAW', b, label, olabel)
        (ph.stores if mode != 'add' else ph.adds).setdefault(b, {})[sid] = label

    def _barrier(self, slot):
        # code the lowering placed before this barrier's arrival (it may have
        # been generated later, for the phase this barrier opens)
        for z, ahead in self.clears.get(slot, ()):
            self.sid += 1
            self._write(z, self.sid, f'clear of {z} before barrier {slot}', 'store', ahead)
        self.ph = _Phase()

    # ---------------------------------------------------------------- run
    def run(self, steps=2):
        """Execute ``steps`` steps of the kernel's event list; returns the races found."""
        low = self.low
        events = _expand(low.trace)
        self.layer = 0
        self.sid = 0
        self.ph = _Phase()
        self.clears = {}
        for ev in low.trace:
            if ev[0] == 'clear' and ev[2] is not None:
                self.clears.setdefault(ev[2], []).append((ev[1], ev[3]))
        for self.step in range(steps):
            self._block(events)
            if self.step + 1 < steps and getattr(low, 'wrap_barrier', True):
                self._barrier(None)
        return self.races

    def _block(self, events):
        cur = None                    # (site id, label, values visible through flags)
        for ev in events:
            kind = ev[0]
            if kind == 'loop':
                _, var, n, body = ev
                for _ in range(n):
                    self._block(body)
                    self.layer += 1
                continue
            if kind == 'barrier':
                self._barrier(ev[2])
                cur = None
                continue
            if kind in ('site', 'flags'):
                self.sid += 1
                visible = frozenset(ev[2]) if kind == 'flags' else frozenset()
                cur = (self.sid, ev[1], visible)
                if kind == 'site':
                    for v in ev[2]:
                        self._read(v, self.sid, ev[1], visible)
                    for v in ev[3]:
                        self._write(v, self.sid, ev[1], self._mode(v))
                self.stored = set()
                continue
            if cur is None:
                self.sid += 1
                cur = (self.sid, f'code after {ev[0]}', frozenset())
                self.stored = set()
            sid, label, visible = cur
            if kind == 'note':
                for v in ev[1]:
                    self._read(v, sid, label, visible)
                for v in ev[2]:
                    self._write(v, sid, label, 'store' if v in self.stored else self._mode(v))
            elif kind == 'store':
                self.stored.add(ev[1])
                # the site's earlier write of it (from its 'site' event) was a plain store
                b = self._buf(ev[1])
                a = self.ph.adds.get(b, {})
                if sid in a:
                    self.ph.stores.setdefault(b, {})[sid] = a.pop(sid)
            elif kind == 'adds':
                for v in ev[2]:
                    self._read(v, sid, label, visible)
                self._write(ev[1], sid, label, 'add')
            elif kind == 'clear':
                _, z, slot, ahead = ev
                if slot is None:
                    self._write(z, sid, f'{label}: clear of {z}', 'store', ahead)
            elif kind == 'feedback':
                _, local, targets = ev
                if not local:
                    for v in targets:
                        self._write(v, sid, 'feedback', 'store')

    def _mode(self, v):
        return 'add' if v in self.fx else 'store'


def check(low, steps=2):
    """Races of lowering ``low`` over ``steps`` steps (empty: every access is ordered)."""
    return PhaseEmulator(low).run(steps)


# ------------------------------------------------------------------ readiness-flag ranges, block by block
def _c_int(expr, env):
    """Value of a C integer expression over non-negative operands: the
    kernel's range bounds, with ``(int)blockIdx.x``, ``(int)nblk`` and the
    names in ``env`` replaced by numbers."""
    import re
    text = expr.replace('(int)blockIdx.x', str(env['blockIdx'])).replace('(int)nblk', str(env['nblk']))
    text = re.sub(r'\b(rl_\w+)\b', lambda m: str(env[m.group(1)]), text)
    if not re.fullmatch(r'[0-9+\-*/%() ]*', text):
        raise ValueError(f'not a plain integer expression: {expr!r}')
    return eval(text.replace('/', '//'), {'__builtins__': {}})     # operands are non-negative: // is C's /


def flag_range_gaps(low):
    """For every readiness-flag wait in ``low.trace``: each consumer block's
    producer blocks, derived from what the consumer reads (a fold split: its
    slice of the fold; an attention point: every query, key and value column
    of its row and head, enumerated over the free axes), must lie in the
    block ranges the kernel waits on (the lowering's C expressions, evaluated
    per block, clamped to the grid as the kernel does). Returns the gaps as
    (site kind, block, missing producer blocks)."""
    gaps = []
    for ev in low.trace:
        if ev[0] != 'flagrange':
            continue
        _, kind, ranges, active, _setup, info = ev
        grid = info['grid']
        for b in range(grid):
            env = {'blockIdx': b, 'nblk': grid}
            if kind == 'split':
                KS, NKB, PPB = info['KS'], info['NKB'], info['PPB']
                q = b % KS
                k0, k1 = q * NKB // KS, (q + 1) * NKB // KS
                need = {p // PPB for p in range(k0 * 32, k1 * 32)}
            else:
                G, PPB, lead, ext = info['G'], info['PPB'], info['lead'], info['ext']
                gi, vals = b % G, {}
                for a, n in zip(reversed(lead), reversed(ext)):
                    vals[a] = gi % n
                    gi //= n
                env.update({f'rl_{a}': v for a, v in vals.items()})
                need = set()
                free = info['free']
                for const, coefs in info['deps']:
                    pts = [const + sum(k * vals[a] for a, k in coefs.items() if a in vals)]
                    for a, k in coefs.items():
                        if a not in vals:
                            pts = [p + k * i for p in pts for i in range(free[a])]
                    need |= {p // PPB for p in pts}
            if not _c_int_bool(active, env):
                continue
            have = set()
            for lo, hi in ranges:
                a0 = _c_int(lo, env)
                a1 = min(_c_int(hi, env), grid - 1)
                have |= set(range(a0, a1 + 1))
            missing = sorted(need - have)
            if missing:
                gaps.append((kind, b, missing))
    return gaps


def _c_int_bool(expr, env):
    import re
    m = re.fullmatch(r'\(int\)blockIdx\.x < (\d+)', expr.strip())
    if not m:
        raise ValueError(f'unexpected activity condition {expr!r}')
    return env['blockIdx'] < int(m.group(1))
