"""Vesta lowering for gfx950: a program -> HIP C++ for ONE persistent kernel
that runs the whole program per launch (one GPT-2 decode step per launch).

    lower(text, res, axis_max, batch=1, per_token=(), outputs=(), feedback=None, timing=False)

Same signature and result type as the reference compiler (reference
``vesta/lower.py:1294``, ``Lowered`` :69-79); the generated source is HIP for
CDNA4 (wave64, 160 KB LDS, agent-scope grid barrier) instead of CUDA.

    res       residue name -> (shape, dtype), dtype 'f32' | 'f16' | 'i32'.
              Shapes as the kernel sees them (batched where per-token);
              scalars have shape () and are read through a pointer.
    axis_max  upper bound of axes whose extent is set at run time (s = t+1)
    batch     B: the program is asked of B tokens at once (batch lift)
    per_token residues that differ per token (x, the key/value cache)
    outputs   named values the host reads; kept in global scratch
    feedback  {'x': 'next', 't': 1}: after the step, x <- next and t += 1,
              so steps run back to back with no host round trip

Pipeline (own design; the placement classes keep the reference's names so a
reader of both can line them up, reference lower.py:21-40):

  batch_lift   every local and per-token residue gains a leading axis 'bt'
  normalise    a bare read of a local with axes becomes a read at its axes
  hoist        a fold that ignores some output axis becomes its own
               statement (the softmax denominator, once per (bt, h))
  alias        carry <- init / carry <- ret / result <- carry share storage
  inline       fold-free values are substituted into their readers unless a
               reader streams a large residue inside its fold
  place        one placement per statement:
    tile     sum whose body reads a residue along its contiguous last axis,
             which is an output axis: 16-byte loads along that axis, rows of
             the fold split over the 4 waves of a block and over blocks
             (split-K); partials reduced in a fixed order by the last block
             to finish the tile, which also runs the epilogue, the statements
             fused into it and the emits it feeds
    lane     sum whose body reads a residue along its contiguous last axis,
             which is the fold axis: a group of lanes per output point,
             16-byte loads along the fold, butterfly reduction
    private  small values every block computes for itself into LDS
    group    consecutive statements that share leading axes and read each
             other only at those axes: one block per leading point
    gridred  a fold over a very long axis into a few points: per-block
             partials, the last block combines them in block order
    thread   one thread per output point, folds as serial loops
  barriers     a grid barrier goes where a statement reads a value written
               since the last barrier, or overwrites one read since then
  codegen      one kernel; the prelude (hip/prelude.h) supplies fp16
               conversion, 16-byte loads, wave64/block reductions, the grid
               barrier and the last-arriver counter

Arithmetic is fp32 with IEEE division and square root and no contraction
of separate multiply and add (elementwise statements round as NumPy does);
the inner products of tile and lane sites use fused multiply-add.
"""
from __future__ import annotations

import math
import re
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from .interp import parse
from .analysis import (BIG, PRIV_SIZE, PRIV_WORK, STAGE_MAX, Analysis, LowerError, batch_lift, replace_node,
                       top_folds)
from .attn import AttnMixin
from .chain import ChainError, ChainMixin
from .ir import defined_names, is_node, stmt_exprs, transform, walk
from .stream import StreamMixin, PREFETCH_VGPRS
from .mfma import MFMA_PIPES, MFMA_ROWS_MIN, MfmaMixin

PRELUDE_PATH = Path(__file__).resolve().parent / 'hip' / 'prelude.h'

WAVE, NWAVE = 64, 8
BLOCK = WAVE * NWAVE          # threads per block: two waves per SIMD, one block per CU
KCAP = 32                     # split-K: at most this many partials per tile column block
GRID_MAX = 1024               # grid reductions keep one partial per block, for up to this many blocks
GRID_WIDE = 256               # blocks per launch: one per CU of an MI355X; from 16 rows on
GRID_DEFAULT = 192            # ... from 4 to 15 rows: a step is a chain of grid barriers, cheaper over
                              # fewer blocks, and 192 keeps two replica blocks per (row, head) of GPT-2
                              # small's attention at B=8 (measured B=8: 331 us per step on 192 blocks,
                              # 345 on 256, 353-355 on 208-240, 429 on 176; B=4: 291 on 192, 305 on 256)
GRID_FEW_ROWS = 144           # ... below 4 rows (measured B=1: 227 us on 144, 233 on 128 and 120, 240 on
                              # 156, 252 on 192, 274 on 96)
LDS_BYTES = 160 * 1024        # LDS of one CU (the kernel runs one block per CU)
REG_MAX = 8                   # register axes: at most this many accumulator rows per lane
PRIV_BUDGET = 16384           # all live private values together: 64 KB of LDS
GROUP_WORK = 1 << 14          # a group statement does at most this much work per leading point
ATTN_WORK = 1 << 17           # ... or this much in a group that streams the key/value cache
LANE_MIN = 32                 # lane-split a fold only if it is at least this long
GRIDRED_MIN = 1 << 14         # grid reduction for a fold at least this long into few points
GRIDRED_POINTS = 8
REPL_MAX = 1 << 14            # points a replicated (every-block) statement may have
PRIV_GROUP = 8                # elementwise private: leading points whose reads are issued together
HOIST_IN_REGISTERS = True     # a private statement over one leading point whose divisors and calls read
                              # only values every wave holds makes them in each thread (no LDS, no block sync)
BTRACE = 96                   # timing: barriers of the last step traced per block
UNROLL = 8                    # rows (tile) / vectors (lane) whose loads are issued together
TILE_LANES = 8                # tile: lanes per row (8 x 16 bytes = one 128-byte line of a weight row)
LINE_WORDS = 32               # one 128-byte line per counter
BAR_WORDS = LINE_WORDS * 10   # grid barrier: 8 per-XCD arrival counters, exit counter, error word
BAR_ERROR = LINE_WORDS * 9 + 1  # the error word (device VH_BAR_ERROR): nonzero once a launch failed
ERR_BARRIER, ERR_RANGE = 1, 2   # ... a grid barrier gave up waiting / an activation beyond fp16 on the matrix cores

FOLD_INIT = {'sum': '0.0f', 'max': '-INFINITY', 'min': 'INFINITY'}
FOLD_OP = {'sum': 'op_sum', 'max': 'op_max', 'min': 'op_min'}
CFUNC = {'exp': 'expf', 'tanh': 'tanhf', 'sqrt': 'sqrtf'}
CTYPE = {'f32': 'float', 'f16': 'vh_half', 'i32': 'int'}
ELEM_BYTES = {'f32': 4, 'f16': 2, 'i32': 4}


@dataclass
class Lowered:
    src: str
    params: list                  # (name, dtype, written) in kernel argument order
    scratch: dict                 # host-visible name -> (offset, axes, static shape)
    scratch_floats: int
    shared_bytes: int             # dynamic LDS per block
    barriers_per_launch: int
    plan: list = field(default_factory=list)      # (statement, placement) for reading
    sites: list = field(default_factory=list)     # timing: label of each timed site (TS is [site][block])
    counters: int = 2                             # length of the bar array
    block: int = BLOCK
    grid_max: int = GRID_MAX
    shapes: dict = field(default_factory=dict)    # residue name -> shape
    name: str = 'vesta_step'                      # the kernel's symbol
    per_cu_max: int = 1                           # resident blocks per CU the kernel is laid out for
    packs: dict = field(default_factory=dict)     # transposed copy -> residue it is made from (at bind)
    history: int = 0                              # tokens a step records in tok_out / reads from tok_in (0: none)


# ------------------------------------------------------------------ AST helpers
# Tree traversal lives in vesta.ir; these names are what the code generators use.
nodes = walk
rebuild = transform
local_names = defined_names


def show(e):
    """Expression -> program-like text (for plans and comments)."""
    if not is_node(e):
        return str(e)
    k = e[0]
    if k == 'num':
        return repr(e[1])
    if k == 'name':
        return e[1]
    if k == 'neg':
        return f'-{show(e[1])}'
    if k == 'call':
        return f'{e[1]}({show(e[2])})'
    if k == 'bin':
        return f'({show(e[2])} {e[1]} {show(e[3])})'
    if k == 'fork':
        return f'fork {show(e[1])} ? {show(e[2])} : {show(e[3])}'
    if k == 'idx':
        return f'{e[1]}[{", ".join(show(i) for i in e[2])}]'
    if k == 'fold':
        return f'fold {e[1]} {e[2]}: {show(e[3])}'
    return str(e)


def show_stmt(s):
    if s[0] == 'let':
        return f'{s[1]}[{", ".join(s[2])}] = {show(s[3])}'
    if s[0] == 'emit':
        return f'residue {s[1]}[{", ".join(show(i) for i in s[2])}] <- {show(s[3])}'
    if s[0] == 'step':
        return f'{s[1]}[{", ".join(s[2])}] = fold step {s[3]}: {show(s[4])} as {s[5]}'
    return str(s)


def c_float(v):
    """A numeric literal as the fp32 constant NumPy would use (weak scalar)."""
    f = float(np.float32(v))
    if math.isinf(f):
        return 'INFINITY' if f > 0 else '-INFINITY'
    txt = repr(f)
    if 'e' not in txt and '.' not in txt:
        txt += '.0'
    return txt + 'f'


# ------------------------------------------------------------------ placements
@dataclass
class Contraction:
    """A sum fold streaming residue W (tile or lane placement)."""
    kind: str                 # 'tile' | 'lane'
    fold: tuple               # the (outermost) fold node
    fold_axes: list           # flattened fold axes, outermost first
    W: str
    widx: list                # W's index expressions
    A: tuple                  # the other factor
    epi: tuple                # the statement's expression with the fold replaced by ('name', '__acc')
    contig: str               # the axis W is contiguous along (output axis j for tile, fold axis for lane)
    reg_axes: list            # output axes W does not depend on
    pt_axes: list             # output axes W depends on (besides contig for tile)
    vec: int = 1



class Lowering(Analysis, StreamMixin, MfmaMixin, AttnMixin, ChainMixin):
    NWAVE, BLOCK, REG_MAX = NWAVE, BLOCK, REG_MAX
    show_stmt = staticmethod(show_stmt)
    nodes_of = staticmethod(nodes)
    rebuild_expr = staticmethod(rebuild)

    def __init__(self, stmts, res, axis_max, outputs, batch, timing=False, grid=None, prefetch_vgprs=None,
                 mfma_pipe=None, local_folds=True):
        self.res = {n: (tuple(int(x) for x in shp), dt) for n, (shp, dt) in res.items()}
        self.axis_max = dict(axis_max or {})
        self.outputs = set(outputs)
        self.batch = batch
        self.timing = timing
        self.static = {}          # axis -> static extent (upper bound for dynamic ones)
        self.dynamic = {}         # axis -> extent expression (run-time)
        self.steps = set()        # step variables
        self.step_ext = {}        # step variable -> loop count
        self.axes_of = {}         # local -> axes
        self.emitted = set()
        self.emit_stmts = []
        self.alias = {}
        self.tmp = 0
        self.plan = []
        self.sites = []
        self.barriers = 0
        self.mult = 1
        self.fresh_id = 0
        self.step_env = {}
        self.fb_targets = set()
        self.inlined = []
        self.grid_auto = grid is None
        self.grid = int(grid or (GRID_FEW_ROWS if batch < 4 else GRID_DEFAULT if batch < 16 else GRID_WIDE))
        self.grid_wide = GRID_WIDE
        self.proj_wider = False       # an attention projection would get its replicas on GRID_WIDE blocks
        self.pf_budget = int(prefetch_vgprs or PREFETCH_VGPRS)   # registers per lane a site may prefetch into
        self.mfma_pipe = int(mfma_pipe or MFMA_PIPES[0])     # k-blocks per register set of an unprefetched MFMA stream
        self.packs = {}           # transposed copy -> the residue it is made from
        self.decls = []           # kernel-scope declarations (prefetch registers)
        self.pf_slots = []        # prefetch code per grid barrier
        self.last_pf = None
        self.loops = []
        self.stage_top = 0
        self.capture = None
        self.in_fold = False          # generating the body of a fold
        self.divr = {}                # shown divisor -> (value, reciprocal) C expressions
        self.invs = {}                # shown subexpression -> C expression of its value
        self.lcap = None              # LDS reads being collected into registers
        self.skip_store = set()       # epilogue values no other statement reads
        self.out_stage = {}           # epilogue value -> (LDS base, points/block, reg axes, point axes)
        self.stream_lds = {}          # value -> (LDS base, points/block, rows) of the site just made
        self.stream_part = {}         # value -> how a stream site split its points over blocks
        self.local_fb = {}            # feedback target -> ('tok', source) | ('inc', k) kept block-local
        self.local_vals = {}          # value -> LDS array every block holds it in (redundant combine)
        self.shared_decls = []        # kernel-scope __shared__ arrays
        self.proj = {}                # id(first attention statement) -> projection it also does
        self.fx = set()               # values kept as 64-bit fixed-point sums in global scratch
        self.elided = set()           # ids of statements another site computes
        self.trace = []               # code-generation events in kernel order, for the phase emulator (vesta.phases)
        self.elided_vals = set()      # values no site stores
        self.scan(stmts)
        stmts = self.normalise(stmts)
        stmts = self.hoist(stmts)
        self.find_aliases(stmts)
        stmts = self.inline(stmts)
        self.stmts = stmts
        self.place_all(stmts)
        self.find_projections(stmts)
        self.peels = {}               # id(step) -> statement of its carry's first value, made where read
        self.peel_active = {}         # carry root -> (loop variable, that statement) inside the loop
        self.find_peels(stmts)
        self.splits = {}              # id(stream statement) -> geometry of its fold split over blocks
        self.local_folds = local_folds
        self.find_splits(stmts)
        self.chains = {}              # id(statement) -> a local fold: its fold over the points its block made
        self.chain_src = {}           # id(the stream making those points) -> the same
        self.chain_local = set()      # values kept only in the LDS of the block that made them
        self.chain_lds = {}           # such a value -> (LDS base, points/block, rows) of the site just made
        self.fx_copies = {}           # fixed-point sum -> copies its adders spread over
        self.flags_off = None         # readiness flag lines in bar (one per block), when a site uses them
        self.fx_parity = {}           # fixed-point sum -> (layer loop variable, its extent): two buffers
        if local_folds:
            self.find_chains(stmts)
            self.find_ready_attn(stmts)
        self.layout(stmts)

    # ------------------------------------------------------------ rewrites
    def find_peels(self, ss):
        """A step loop whose carry starts from a replicated statement (one
        reading residues only): in the first iteration, reads of the carry
        evaluate that statement where they are, so it is never stored (every
        block would otherwise write the same values to the same addresses)."""
        for i, s in enumerate(ss):
            if s[0] != 'step':
                continue
            self.find_peels(s[6])
            _, name, axes, var, init, carry, blk = s
            if init[0] != 'idx' or self.alias.get(init[1]) != carry or var in self.dynamic:
                continue
            if self.static.get(var, 0) < 1:
                continue
            defs = [t for t in ss[:i] if t[0] == 'let' and t[1] == init[1]]
            if len(defs) != 1 or self.place.get(id(defs[0])) != 'repl':
                continue
            if self.readers_of.get(init[1], set()) != {id(s)}:
                continue
            self.peels[id(s)] = defs[0]
            self.elided.add(id(defs[0]))

    def peel_value(self, r, ix):
        """For a carry read in the first iteration of its loop: C text of
        its first value at the index ix (C expressions), or None."""
        pk = self.peel_active.get(r)
        if pk is None:
            return None
        lv, zs = pk
        env = {a: (c, 'int') for a, c in zip(zs[2], ix)}
        saved, self.capture = self.capture, None
        try:
            pre = []
            v, t = self.expr(zs[3], env, pre, '')
        finally:
            self.capture = saved
        if pre:
            raise LowerError(f'first value of {r} needs statements of its own')
        return lv, self.as_float(v, t)

    # ------------------------------------------------------------ placement
    def _place_block(self, ss):
        i = 0
        made, made_axes = set(), None      # results of the last contraction and its epilogue
        while i < len(ss):
            s = ss[i]
            if s[0] == 'step':
                self._place_block(s[6])
                made = set()
                i += 1
                continue
            if s[0] != 'let':
                i += 1
                continue
            run = self.attn_run(ss, i)
            if run:
                lead, members = run
                self.groups[id(members[0])] = (lead, members)
                ids = {id(t) for t in members}
                self.group_local[id(members[0])] = [
                    t[1] for t in members
                    if t[1] not in self.outputs and not (self.readers_of.get(t[1], set()) - ids)]
                for t in members:
                    self.place[id(t)] = 'group'
                    self.in_group.add(id(t))
                made = set()
                i += len(members)
                continue
            c = self.contraction(s)
            if c is not None:
                self.place[id(s)] = c.kind
                self.info[id(s)] = c
                made, made_axes = {s[1]}, list(s[2])
                i += 1
                continue
            if made and self.epilogue_ok(s, made, made_axes):
                # an elementwise statement right after a contraction runs in its epilogue
                self.place[id(s)] = 'epilogue'
                made.add(s[1])
                i += 1
                continue
            made = set()
            if self.priv_ok(s):
                self.place[id(s)] = 'private'
                self.private.add(s[1])
                i += 1
                continue
            g = self.gridred(s)
            if g:
                self.place[id(s)] = 'gridred'
                if i + 1 < len(ss) and self.argmin_of_max(s, ss[i + 1]):
                    # max and lowest index of the max: one grid reduction of (value, index) pairs
                    self.place[id(s)] = 'argmax'
                    self.place[id(ss[i + 1])] = 'argmax'
                    self.argmax[id(s)] = ss[i + 1]
                    i += 2
                    continue
                i += 1
                continue
            run = self.group_run(ss, i)
            if run:
                lead, members = run
                self.groups[id(members[0])] = (lead, members)
                for t in members:
                    self.place[id(t)] = 'group'
                    self.in_group.add(id(t))
                i += len(members)
                continue
            if self.block_ok(s):
                self.groups[id(s)] = (list(s[2]), [s])
                self.place[id(s)] = 'group'
                self.in_group.add(id(s))
                i += 1
                continue
            self.place[id(s)] = 'repl' if self.repl_ok(s) else 'thread'
            i += 1

    def repl_ok(self, s):
        """A small statement that reads only residues is computed by every
        block for every point (so no block waits for another to read it)."""
        if s[0] != 'let' or top_folds(s[3]) or s[1] in self.outputs:
            return False
        if any(a in self.dynamic for a in s[2]) or self.size(s[2]) > REPL_MAX:
            return False
        if self.reads(s[3]) - set(self.res):
            return False
        return not any(n[1] in self.emitted for n in self.res_reads(s[3]))

    def epilogue_ok(self, s, made, axes):
        if list(s[2]) != axes or top_folds(s[3]) or s[1] in self.alias or s[1] in set(self.alias.values()):
            return False
        same = [('name', a) for a in axes]
        hits = [n for n in nodes(s[3]) if n[0] == 'idx' and n[1] in made]
        return bool(hits) and all(list(n[2]) == same for n in hits)

    def block_ok(self, s):
        """A long fold into many points: one block per point."""
        e = s[3]
        return (e[0] == 'fold' and s[2] and not any(a in self.dynamic for a in s[2])
                and self.static[e[2]] >= 1024 and not self.big_reads(e)
                and s[1] not in self.alias and s[1] not in set(self.alias.values()))

    def attn_run(self, ss, i):
        """Consecutive statements sharing leading axes that stream the
        key/value cache (contractions over emitted residues) and read each
        other only at the leading point: one block per leading point."""
        s = ss[i]
        if s[0] != 'let' or len(s[2]) < 2:
            return None
        carries = set(self.alias.values())
        for plen in range(len(s[2]) - 1, 0, -1):
            lead = list(s[2][:plen])
            if any(a in self.dynamic for a in lead):
                continue
            same = [('name', a) for a in lead]
            run, names, has_c = [], set(), False
            for t in ss[i:]:
                if t[0] != 'let' or len(t[2]) < plen or list(t[2][:plen]) != lead:
                    break
                if t[1] in self.alias or t[1] in carries or self.big_reads(t[3]):
                    break
                if any(n[0] == 'idx' and n[1] in names and list(n[2][:plen]) != same for n in nodes(t[3])):
                    break
                if self.size(t[2][plen:]) * self.fold_work(t[3]) > ATTN_WORK:
                    break
                c = self.contraction(t)
                if c is not None:
                    if not self.block_contraction_ok(c, t, plen):
                        break
                    has_c = True
                run.append(t)
                names.add(t[1])
            if len(run) >= 2 and has_c:
                return lead, run
        return None

    def block_contraction_ok(self, c, t, plen):
        rest = list(t[2][plen:])
        if c.reg_axes:
            return False
        if c.kind == 'lane':
            return True
        return rest == [c.contig] and c.contig not in self.dynamic

    def group_ok(self, t, plen):
        return (t[0] == 'let' and not self.big_reads(t[3]) and self.contraction(t) is None
                and not self.priv_ok(t) and len(t[2]) >= plen
                and not any(a in self.dynamic for a in t[2][:plen])
                and self.size(t[2][plen:]) * self.fold_work(t[3]) <= GROUP_WORK
                and t[1] not in self.alias and t[1] not in set(self.alias.values()))

    def group_run(self, ss, i):
        s = ss[i]
        for plen in range(len(s[2]), 0, -1):
            if not self.group_ok(s, plen):
                continue
            lead = list(s[2][:plen])
            run, names = [s], {s[1]}
            for t in ss[i + 1:]:
                if t[0] != 'let' or list(t[2][:plen]) != lead or not self.group_ok(t, plen):
                    break
                bad = False
                for n in nodes(t[3]):
                    if n[0] == 'idx' and n[1] in names and list(n[2][:plen]) != [('name', a) for a in lead]:
                        bad = True
                if bad:
                    break
                run.append(t)
                names.add(t[1])
            if len(run) >= 2:
                return lead, run
        return None

    def argmin_of_max(self, s1, s2):
        """s2 = fold min n: fork E[n] == s1 ? n : C, with s1 = fold max n: E[n]."""
        e1, e2 = s1[3], s2[3]
        if s2[0] != 'let' or list(s2[2]) != list(s1[2]) or e1[1] != 'max' or e2[0] != 'fold' or e2[1] != 'min' \
                or e2[2] != e1[2] or s2[1] in self.alias or s1[1] in self.alias:
            return False
        body = e2[3]
        if body[0] != 'fork' or body[2] != ('name', e1[2]) or body[3][0] != 'num':
            return False
        cond = body[1]
        me = ('idx', s1[1], [('name', a) for a in s1[2]]) if s1[2] else ('name', s1[1])
        return cond[0] == 'bin' and cond[1] == '==' and (
            (cond[2] == e1[3] and cond[3] == me) or (cond[3] == e1[3] and cond[2] == me))

    def gridred(self, s):
        e = s[3]
        if e[0] != 'fold' or self.size(s[2]) > GRIDRED_POINTS or any(a in self.dynamic for a in s[2]):
            return False
        return e[2] in self.static and e[2] not in self.dynamic and self.static[e[2]] >= GRIDRED_MIN

    def contraction(self, s):
        """Tile or lane pattern of a let statement, or None."""
        if s[0] != 'let':
            return None
        name, axes, e = s[1], list(s[2]), s[3]
        tops = top_folds(e)
        if len(tops) != 1 or tops[0][1] != 'sum':
            return None
        fold = tops[0]
        fold_axes, body = [fold[2]], fold[3]
        while body[0] == 'fold' and body[1] == 'sum':
            fold_axes.append(body[2])
            body = body[3]
        if body[0] != 'bin' or body[1] != '*':
            return None
        if any(a in axes for a in fold_axes) or len(set(fold_axes)) != len(fold_axes):
            return None
        if any(not self.is_axis(a) for a in fold_axes):
            return None
        epi = replace_node(e, fold, ('name', '__acc'))
        if '__acc' not in [n[1] for n in nodes(epi) if n[0] == 'name']:
            return None
        for W_node, A in ((body[3], body[2]), (body[2], body[3])):
            if W_node[0] != 'idx' or W_node[1] not in self.res:
                continue
            W, widx = W_node[1], W_node[2]
            shape, dt = self.res[W]
            if dt not in ('f16', 'f32') or len(shape) != len(widx) or not shape:
                continue
            last = widx[-1]
            if last[0] != 'name':
                continue
            contig = last[1]
            others = set()
            for x in widx[:-1]:
                others |= self.free_axes(x)
            if contig in others:
                continue
            w_axes = others | {contig}
            a_free = self.free_axes(A) - set(fold_axes)
            if not a_free <= set(axes):
                continue
            if not (self.free_axes(epi) - {'__acc'}) <= set(axes):
                continue
            reg = [a for a in axes if a not in w_axes]
            pt = [a for a in axes if a in w_axes and a != contig]
            if any(a in self.dynamic for a in reg):
                continue
            vec_for = {'f16': (8, 4, 2), 'f32': (4, 2)}[dt]
            if contig in axes and len(fold_axes) >= 1 and contig not in fold_axes:
                # tile: contiguous along an output axis
                if contig in self.dynamic or contig in self.free_axes(A):
                    continue
                J = self.static[contig]
                vec = next((v for v in vec_for if J % v == 0 and shape[-1] % v == 0), 1)
                if self.size(reg) > 64:
                    continue
                return Contraction('tile', fold, fold_axes, W, widx, A, epi, contig, reg, pt, vec)
            if len(fold_axes) == 1 and contig == fold_axes[0]:
                # lane: contiguous along the fold axis
                if contig in self.dynamic or self.static[contig] < LANE_MIN:
                    continue
                K = self.static[contig]
                vec = next((v for v in vec_for if K % v == 0 and shape[-1] % v == 0), 1)
                if self.size(reg) > 64:
                    continue
                return Contraction('lane', fold, fold_axes, W, widx, A, epi, contig, reg, pt, vec)
        return None

    # ------------------------------------------------------------ storage
    def private_spans(self, ss):
        """Live span (position of the defining statement, last position that
        needs it) of every private value, positions counted over the
        statements in program order with loop bodies inlined once.

        A value made before a step loop and needed from the loop's first
        position on is needed by every iteration, so its span reaches the
        loop's end (the position after the body's last statement); loops are
        visited innermost first, in program order. Values made inside a loop
        are made again by every iteration and keep their own span."""
        stmts, loops = [], []          # flattened statements; (first, end) of every loop, innermost first

        def visit(block):
            for s in block:
                if s[0] != 'step':
                    stmts.append(s)
                    continue
                first = len(stmts)
                visit(s[6])
                loops.append((first, len(stmts)))
        visit(ss)
        made, need = {}, {}
        for pos, s in enumerate(stmts):
            if s[0] == 'let' and s[1] in self.private and s[1] not in made:
                made[s[1]] = need[s[1]] = pos
            for n in {n for e in stmt_exprs(s) for n in self.reads(e)} & made.keys():
                need[n] = pos
        for first, end in loops:
            for n, pos in made.items():
                if pos < first <= need[n]:
                    need[n] = max(need[n], end)
        return {n: (made[n], need[n]) for n in made}

    @staticmethod
    def lowest_gap(busy, size, align=4):
        """Lowest offset (a multiple of ``align`` floats, or 0) where ``size``
        floats fit between the address ranges in ``busy`` ((offset, size)
        pairs that do not overlap each other)."""
        at = 0
        for off, n in sorted(busy):
            if at + size <= off:
                return at
            at = max(at, (off + n + align - 1) // align * align)
        return at

    def layout(self, ss):
        """Global scratch for values shared across blocks; LDS for private
        values, each given the lowest free range (16-byte aligned, for vector
        LDS reads) among the values still live when it is made, in the order
        they are made."""
        spans = self.private_spans(ss)
        self.lds, placed, top = {}, [], 0        # placed: (span end, LDS offset, floats)
        for n in sorted(spans, key=lambda v: spans[v][0]):
            born, dies = spans[n]
            size = self.size(self.axes_of[n])
            placed = [p for p in placed if p[0] >= born]
            off = self.lowest_gap([(o, k) for _, o, k in placed], size)
            if off + size > PRIV_BUDGET:
                raise LowerError(f'private values exceed the LDS budget at {n}')
            placed.append((dies, off, size))
            self.lds[n] = off
            top = max(top, off + size)
        self.lds_floats = -(-top // 4) * 4
        self.g, self.goff = {}, 0
        for n in self.axes_of:
            r = self.root(n)
            if r in self.private or r in self.g or n in self.inlined or r in self.elided_vals:
                continue
            self.g[r] = self.goff
            words = (self.fx_words(r) * (2 if r in self.fx_parity else 1) if r in self.fx
                     else max(1, self.size(self.axes_of[r])))
            self.goff += -(-words // LINE_WORDS) * LINE_WORDS
        self.counters = BAR_WORDS
        self.staged = {}
        self.glocal = {}
        self.stage_floats = 0

    def alloc_scratch(self, n):
        off = self.goff
        self.goff += -(-n // LINE_WORDS) * LINE_WORDS
        return off

    def alloc_counters(self, n):
        """n counters, one 128-byte line each; counter i is at offset + i * LINE_WORDS."""
        off = self.counters
        self.counters += n * LINE_WORDS
        return off

    def strides(self, axes):
        st, acc = [], 1
        for a in reversed(axes):
            st.append(acc)
            acc *= self.static[a]
        return list(reversed(st))

    # ------------------------------------------------------------ expressions
    def fresh(self, base):
        self.fresh_id += 1
        return f'{base}{self.fresh_id}'

    def expr(self, e, env, out, ind):
        """C code of e as (text, type); type is 'int', 'float' or 'bool'.
        Folds inside e become serial loops appended to ``out``."""
        k = e[0]
        if self.invs and k in ('call', 'bin'):
            got = self.invs.get(show(e))
            if got is not None:
                return got, 'float'
        if k == 'num':
            v = e[1]
            if isinstance(v, int) and not isinstance(v, bool):
                return str(v), 'int'
            return c_float(v), 'float'
        if k == 'name':
            n = e[1]
            if n in env:
                return env[n]
            if n in self.step_env:
                return self.step_env[n]
            if n in self.axes_of:
                if self.axes_of[n]:
                    raise LowerError(f'{n} read without its axes')
                return self.load(n, []), 'float'
            if n in self.res:
                shape, dt = self.res[n]
                if math.prod(shape) != 1:
                    raise LowerError(f'residue {n} read without an index')
                if n in self.emitted:
                    return self.res_value(n, '0')
                return f'rs_{n}', ('int' if dt == 'i32' else 'float')
            if n in self.static:
                raise LowerError(f'axis {n} is not bound here')
            raise NameError(n)
        if k == 'neg':
            a, t = self.expr(e[1], env, out, ind)
            return f'(-{self.as_num(a, t)})', ('int' if t == 'int' else 'float')
        if k == 'call':
            a, t = self.expr(e[2], env, out, ind)
            return f'{CFUNC[e[1]]}({self.as_float(a, t)})', 'float'
        if k == 'bin':
            op = e[1]
            a, ta = self.expr(e[2], env, out, ind)
            if op == '/' and self.divr and show(e[3]) in self.divr:
                # a divisor that does not vary over the points being made:
                # its value and reciprocal were computed once
                dv, rv = self.divr[show(e[3])]
                return f'vh_divr({self.as_float(a, ta)}, {dv}, {rv})', 'float'
            b, tb = self.expr(e[3], env, out, ind)
            if op in ('==', '<', '>', '<=', '>='):
                if ta == 'int' and tb == 'int':
                    return f'({a} {op} {b})', 'bool'
                return f'({self.as_float(a, ta)} {op} {self.as_float(b, tb)})', 'bool'
            if op == '/':
                if e[3][0] == 'num' and np.isfinite(np.float32(e[3][1])) and np.float32(e[3][1]) != 0:
                    c = np.float32(e[3][1])
                    r = np.float32(1.0) / c
                    if np.frexp(c)[0] in (0.5, -0.5):
                        # a power of two: the reciprocal is exact
                        return f'({self.as_float(a, ta)} * {c_float(r)})', 'float'
                    return f'vh_divr({self.as_float(a, ta)}, {c_float(c)}, {c_float(r)})', 'float'
                return f'({self.as_float(a, ta)} / {self.as_float(b, tb)})', 'float'
            if ta == 'int' and tb == 'int':
                return f'({a} {op} {b})', 'int'
            return f'({self.as_float(a, ta)} {op} {self.as_float(b, tb)})', 'float'
        if k == 'fork':
            c, tc = self.expr(e[1], env, out, ind)
            a, ta = self.expr(e[2], env, out, ind)
            b, tb = self.expr(e[3], env, out, ind)
            cond = c if tc == 'bool' else f'({self.as_float(c, tc)} != 0.0f)'
            if ta == 'int' and tb == 'int':
                return f'({cond} ? {a} : {b})', 'int'
            return f'({cond} ? {self.as_float(a, ta)} : {self.as_float(b, tb)})', 'float'
        if k == 'idx':
            n = e[1]
            ix = [self.index(x, env, out, ind) for x in e[2]]
            if n in self.res:
                shape = self.res[n][0]
                if len(ix) != len(shape):
                    raise LowerError(f'residue {n} has {len(shape)} axes, indexed with {len(ix)}')
                ix = [self.clamp(i, x, d) for i, x, d in zip(ix, e[2], shape)]
                return self.res_value(n, self.addr(ix, self.res_strides(n)))
            if n in self.axes_of:
                if len(ix) != len(self.axes_of[n]):
                    raise LowerError(f'{n} has axes {self.axes_of[n]}, indexed with {len(ix)}')
                return self.load(n, ix), 'float'
            raise NameError(n)
        if k == 'fold':
            op, ax, body = e[1], e[2], e[3]
            if ax not in self.static:
                raise ValueError(f'fold over unknown axis {ax}')
            saved_cap, self.capture = self.capture, None
            try:
                return self.expr_fold(e, env, out, ind)
            finally:
                self.capture = saved_cap
        raise LowerError(f'cannot lower {e}')

    def expr_fold(self, e, env, out, ind):
        if True:
            op, ax, body = e[1], e[2], e[3]
            acc = self.fresh('acc')
            kv = self.fresh(f'k_{ax}_')
            out.append(f'{ind}float {acc} = {FOLD_INIT[op]};')
            out.append(f'{ind}#pragma unroll 8')
            out.append(f'{ind}for (int {kv} = 0; {kv} < {self.ext_c(ax)}; ++{kv}) {{')
            inner = []
            saved, self.lcap = self.lcap, None       # reads in the loop stay in the loop
            try:
                v, t = self.expr(body, {**env, ax: (kv, 'int')}, inner, ind + '  ')
            finally:
                self.lcap = saved
            out += inner
            out.append(f'{ind}  {acc} = {FOLD_OP[op]}({acc}, {self.as_float(v, t)});')
            out.append(f'{ind}}}')
            return acc, 'float'

    def as_float(self, a, t):
        if t == 'float':
            return a
        return f'((float){a})'

    def as_num(self, a, t):
        return f'((float){a})' if t == 'bool' else a

    def index(self, e, env, out, ind):
        v, t = self.expr(e, env, out, ind)
        if t == 'int':
            return v
        if t == 'float' and e[0] == 'idx' and e[1] in self.axes_of:
            return f'((int){v})'
        raise LowerError(f'index {show(e)} is not an integer')

    def data_dependent(self, e):
        """Does index expression e depend on stored data (not only on axes)?"""
        return any(n[0] == 'idx' or (n[0] == 'name' and (n[1] in self.res or n[1] in self.axes_of))
                   for n in nodes(e))

    def clamp(self, i, e, dim):
        """An index computed from data is kept inside the residue, so a bad
        token id or position cannot read or write outside the buffer."""
        if not self.data_dependent(e):
            return i
        return f'min(max({i}, 0), {dim - 1})'

    def addr(self, ix, strides):
        terms = []
        for i, s in zip(ix, strides):
            if i == '0':
                continue
            terms.append(i if s == 1 else f'({i}) * {s}')
        return ' + '.join(terms) if terms else '0'

    def res_strides(self, n):
        shape = self.res[n][0]
        st, acc = [], 1
        for d in reversed(shape):
            st.append(acc)
            acc *= d
        return list(reversed(st))

    def coherent(self, n):
        """Residues written during a launch (emits, feedback targets) are
        read and written through the coherent path."""
        return n in self.emitted or n in self.fb_targets

    def res_value(self, n, addr):
        dt = self.res[n][1]
        if n in self.local_fb:
            kind = self.local_fb[n][0]
            return (f'xfb_{n}[{addr}]' if kind == 'tok' else f'tlv_{n}'), 'int'
        if self.coherent(n):
            if dt == 'f16':
                return f'ldc_h(rb_{n}, {addr})', 'float'
            if dt == 'f32':
                return f'ldc(R_{n} + {addr})', 'float'
            return f'ldc_i(R_{n} + {addr})', 'int'
        rr = self.rsrc(n)
        if dt == 'f16':
            return self.captured(f'ldg_h({rr}, {addr})', raw=(f'ldg_raw16({rr}, {addr})', 'unsigned short', 'h2f')), 'float'
        if dt == 'f32':
            return self.captured(f'ldg_f({rr}, {addr})'), 'float'
        return self.captured(f'ldg_i({rr}, {addr})', 'int'), 'int'

    def rsrc(self, n):
        """Buffer descriptor over residue n."""
        shape, dt = self.res[n]
        nbytes = max(1, math.prod(shape)) * ELEM_BYTES[dt]
        if nbytes >= 1 << 32:
            raise LowerError(f'residue {n} is {nbytes} bytes; buffer access is limited to 4 GiB')
        return f'mk_rsrc(R_{n}, {nbytes}u)'

    def captured(self, text, kind='float', root=None, raw=None):
        """Inside a capture (code generated for a site whose loads are issued
        early, at its barrier), a load becomes a register filled there; loads
        of values that may be written after that point stay in place."""
        cap = self.capture
        if cap is None or (root is not None and (root in cap['unsafe'] or root in self.dirty)):
            return text
        if any(re.search(r'\b' + re.escape(v) + r'\b', text) for v in cap.get('forbid', ())):
            return text
        dd = cap.get('dedupe')
        if dd is not None and text in dd:
            return dd[text]
        name = f"{cap['prefix']}{len(cap['loads'])}"
        if raw is not None:
            # keep the loaded bits; convert where the value is used, so nothing
            # waits for the load where it is issued
            load, ctype, conv = raw
            cap['loads'].append((name, load, ctype))
            use = f'{conv}({name})'
        else:
            cap['loads'].append((name, text, kind))
            use = name
        if dd is not None:
            dd[text] = use
        return use

    def load(self, n, ix):
        """A local: LDS if private or staged, else a coherent load of global scratch."""
        r = self.root(n)
        a = self.addr(ix, self.strides(self.axes_of[r]))
        if r in self.private:
            return self.lds_read(f'sh_f[{self.lds[r]} + {a}]')
        if r in self.staged:
            return self.lds_read(f'sh_f[{self.staged[r]} + {a}]')
        if r in self.glocal:
            off, plen = self.glocal[r]
            return self.lds_read(f'sh_f[{off} + {self.addr(ix[plen:], self.strides(self.axes_of[r][plen:]))}]')
        pv = self.peel_value(r, ix)
        if r in self.fx_copies:
            i = f'{self.gofs(r)} + 2u * ({a})'
            v = f'fxld_c<{self.fx_copies[r]}>(rb_S, {i}, {self.fx_copy_stride(r)}u)'
            return f'({pv[0]} == 0 ? {pv[1]} : {v})' if pv is not None else self.captured(v, 'float', r)
        if r in self.fx:
            i = f'{self.gofs(r)} + 2u * ({a})'
            if pv is not None:
                return f'({pv[0]} == 0 ? {pv[1]} : fxld(rb_S, {i}))'
            return self.captured(f'fxld(rb_S, {i})', 'float', r, raw=(f'ldfx_raw(rb_S, {i})', 'long long', 'vh_fx2f'))
        if pv is not None:
            return f'({pv[0]} == 0 ? {pv[1]} : ldcs(rb_S, {self.g[r]} + {a}))'
        return self.captured(f'ldcs(rb_S, {self.g[r]} + {a})', 'float', r)

    def store(self, n, ix, v, t):
        r = self.root(n)
        a = self.addr(ix, self.strides(self.axes_of[r]))
        if r in self.private:
            return f'sh_f[{self.lds[r]} + {a}] = {self.as_float(v, t)};'
        if r in self.glocal:
            off, plen = self.glocal[r]
            return f'sh_f[{off} + {self.addr(ix[plen:], self.strides(self.axes_of[r][plen:]))}] = {self.as_float(v, t)};'
        if r in self.fx_copies or r in self.fx_parity:
            raise LowerError(f'{r} is a fixed-point sum in copies or parity buffers: only atomic adds go into it')
        if r in self.fx:
            return f'fxst(rb_S, {self.g[r]} + 2u * ({a}), {self.as_float(v, t)});'
        return f'stcs(rb_S, {self.g[r]} + {a}, {self.as_float(v, t)});'

    def decode(self, var, axes, out, ind, prefix='i_'):
        """Lines binding prefix+axis for each axis from flat index ``var``
        (last axis fastest); returns the env entries."""
        env = {}
        if not axes:
            return env
        if len(axes) == 1:
            out.append(f'{ind}const int {prefix}{axes[0]} = {var};')
            env[axes[0]] = (f'{prefix}{axes[0]}', 'int')
            return env
        rem = self.fresh('r')
        out.append(f'{ind}int {rem} = {var};')
        for a in reversed(axes[1:]):
            out.append(f'{ind}const int {prefix}{a} = {rem} % {self.ext_c(a)}; {rem} /= {self.ext_c(a)};')
            env[a] = (f'{prefix}{a}', 'int')
        out.append(f'{ind}const int {prefix}{axes[0]} = {rem};')
        env[axes[0]] = (f'{prefix}{axes[0]}', 'int')
        return env

    def count_c(self, axes):
        if not axes:
            return '1'
        return ' * '.join(self.ext_c(a) for a in axes)

    # ------------------------------------------------------------ hazards
    def root_reads(self, exprs, exclude=()):
        out = set()
        for e in exprs:
            for n in self.reads(e):
                if n in exclude:
                    continue
                out.add(self.root(n) if n in self.axes_of else n)
        return out

    def sync(self, reads, writes, out, ind, what):
        """Grid barrier if a read sees a value written since the last barrier
        or a write overwrites one read since then (by another site)."""
        gl_reads = {n for n in reads if n not in self.private}
        gl_writes = {n for n in writes if n not in self.private}
        if (gl_reads & self.dirty) or (gl_writes & self.readers) or (gl_writes & self.dirty):
            self.barrier(out, ind, what)
        if not getattr(self, 'first_barrier', True):
            self.head_io[0] |= gl_reads
            self.head_io[1] |= gl_writes
        self.readers |= gl_reads
        self.trace.append(('site', what, frozenset(gl_reads), frozenset(gl_writes)))

    def barrier(self, out, ind, what='', pre_wait=()):
        self.trace.append(('barrier', what, len(self.pf_slots)))
        out.append(f'{ind}/*@PZ{len(self.pf_slots)}@*/')   # code that must end before the arrival
        out.append(f'{ind}bk_ += 1u; grid_arrive(bar);' + (f'  // before {what}' if what else ''))
        self.mark(out, ind, f'arrive before {what}')
        if self.timing:
            # the launch's last step: each block's arrival and release time at every barrier
            out.append(f'{ind}if (tid == 0 && st_ + 1 == nsteps && bk_ - bk0_ <= {BTRACE}u) '
                       f'TS[TSB_ + (bk_ - bk0_ - 1u) * 2u * nblk + blockIdx.x] = vh_clock();')
        out += [ind + x for x in pre_wait]
        self.pf_open(out, ind, self.dirty, self.readers)
        out.append(f'{ind}grid_wait(bar, nblk, bk_);')
        if self.timing:
            out.append(f'{ind}if (tid == 0 && st_ + 1 == nsteps && bk_ - bk0_ <= {BTRACE}u) '
                       f'TS[TSB_ + ((bk_ - bk0_ - 1u) * 2u + 1u) * nblk + blockIdx.x] = vh_clock();')
        if self.loops:
            self.loops[-1]['body_barrier'] = True
        self.first_barrier = True
        self.barriers += self.mult
        self.dirty, self.readers = set(), set()
        self.mark(out, ind, f'barrier before {what}')

    def mark(self, out, ind, label):
        if self.timing is not True:
            # a site boundary the compiler keeps: code is not scheduled across
            # it, which keeps register live ranges inside their site
            out.append(f'{ind}asm volatile("");')
            return
        k = len(self.sites)
        if k >= 1024:
            return
        self.sites.append(label)
        out.append(f'{ind}if (tid == 0) {{ unsigned long long tn_ = vh_clock(); ts_sh[{k}] += tn_ - tlast_; '
                   f'tlast_ = tn_; }}')

    # ------------------------------------------------------------ statements
    def gen(self, ss, out, ind):
        i = 0
        while i < len(ss):
            s = ss[i]
            k = s[0]
            if k in ('axis', 'recv', 'ret'):
                i += 1
                continue
            if self.place.get(id(s)) != 'argmax':
                self.stream_lds = {}      # the LDS copy of a stream's values lasts until its next site
            if k == 'step':
                self.gen_step(s, out, ind)
                i += 1
                continue
            if k == 'emit':
                self.gen_emit(s, out, ind)
                i += 1
                continue
            if id(s) in self.elided:
                i += 1
                continue
            if id(s) in self.groups:
                lead, members = self.groups[id(s)]
                at = self.attn_of(lead, members)
                if at is not None:
                    self.gen_attn(at, out, ind, self.proj.get(id(s)))
                else:
                    self.gen_group(lead, members, out, ind)
                i += len(members)
                continue
            p = self.place[id(s)]
            if p == 'private':
                run = [s]
                while i + len(run) < len(ss) and ss[i + len(run)][0] == 'let' \
                        and self.place.get(id(ss[i + len(run)])) == 'private':
                    run.append(ss[i + len(run)])
                self.gen_private(run, out, ind, self.base_after(ss, i + len(run)))
                i += len(run)
                continue
            if id(s) in self.chains:
                self.gen_chain(s, self.chains[id(s)], out, ind)
                i += 1
                continue
            if id(s) in self.splits:
                self.gen_stream_split(s, self.splits[id(s)], out, ind)
                i += 1
                continue
            if p in ('tile', 'lane'):
                fused = self.fusable(ss, i)
                st = self.stream_of(self.info[id(s)])
                if st is not None:
                    self.gen_stream(s, self.info[id(s)], st, fused, out, ind)
                elif p == 'tile':
                    self.gen_tile(s, self.info[id(s)], fused, out, ind)
                else:
                    self.gen_lane(s, self.info[id(s)], fused, out, ind)
                i += 1 + len(fused)
                continue
            if p == 'argmax':
                self.gen_argmax(s, self.argmax[id(s)], out, ind)
                i += 2
                continue
            if p == 'gridred':
                self.gen_gridred(s, out, ind)
            elif p == 'repl':
                self.gen_repl(s, out, ind)
            else:                   # thread, or an epilogue statement its contraction could not take
                self.gen_thread(s, out, ind)
            i += 1

    # -- fusion into an epilogue
    def fusable(self, ss, i):
        """Statements right after contraction ss[i] that its epilogue can run:
        same-point elementwise lets and emits whose value reads the result at
        an invertible affine index."""
        s = ss[i]
        axes = list(s[2])
        made = {s[1]}
        fused = []
        for t in ss[i + 1:]:
            if t[0] == 'let':
                if (list(t[2]) != axes or top_folds(t[3]) or self.place.get(id(t)) in ('private', 'group')
                        or id(t) in self.groups or t[1] in self.private):
                    break
                ok = True
                for n in nodes(t[3]):
                    if n[0] == 'idx' and n[1] in made and list(n[2]) != [('name', a) for a in axes]:
                        ok = False
                    if n[0] in ('name', 'idx') and n[1] not in made:
                        nm = n[1]
                        r = self.root(nm) if nm in self.axes_of else nm
                        if r in self.dirty or (nm in self.emitted):
                            ok = False
                if not ok or self.root(t[1]) in self.readers:
                    break
                fused.append(('let', t, None))
                made.add(t[1])
                continue
            if t[0] == 'emit':
                inv = self.emit_inverse(t, made, axes)
                if inv is None:
                    break
                fused.append(('emit', t, inv))
                continue
            break
        return fused

    def emit_inverse(self, t, made, axes):
        """For an emit whose value reads one value made here at an affine
        index of the emit's axes: how to recover those axes from the point."""
        reads = [n for n in nodes(t[3]) if n[0] == 'idx' and n[1] in made]
        if len(reads) != 1 or any(n[0] == 'name' and n[1] in made for n in nodes(t[3])):
            return None
        src = reads[0]
        for e in t[2]:
            if any(n[0] in ('name', 'idx') and n[1] in made for n in nodes(e)):
                return None
        e_axes = set()
        for e in list(t[2]) + [t[3]]:
            e_axes |= self.free_axes(e)
        e_axes = [a for a in e_axes if self.is_axis(a)]
        for n in nodes(t[3]):
            if n[0] in ('name', 'idx') and n[1] not in made:
                nm = n[1]
                r = self.root(nm) if nm in self.axes_of else nm
                if r in self.dirty or nm in self.emitted:
                    return None
        # each position of the source index: an affine form over emit axes
        plan = []
        seen = set()
        for pos, ie in enumerate(src[2]):
            aff = self.affine(ie)
            if aff is None:
                return None
            const, coefs = aff
            for a in coefs:
                if a not in e_axes or a in seen:
                    return None
                seen.add(a)
            terms = sorted(coefs.items(), key=lambda kv: kv[1])
            radix = 1
            for a, c in terms:
                if c != radix or a in self.dynamic:
                    return None
                radix *= self.static[a]
            plan.append((axes[pos], const, [a for a, _ in reversed(terms)], radix))
        if set(e_axes) != seen:
            return None
        return src, plan

    def affine(self, e):
        """(const, {axis: coef}) if e is an integer affine form of axes."""
        k = e[0]
        if k == 'num':
            return (int(e[1]), {}) if isinstance(e[1], int) else None
        if k == 'name':
            return (0, {e[1]: 1}) if self.is_axis(e[1]) else None
        if k == 'bin' and e[1] in ('+', '-'):
            a, b = self.affine(e[2]), self.affine(e[3])
            if a is None or b is None:
                return None
            sg = 1 if e[1] == '+' else -1
            coefs = dict(a[1])
            for n, c in b[1].items():
                coefs[n] = coefs.get(n, 0) + sg * c
            return a[0] + sg * b[0], {n: c for n, c in coefs.items() if c}
        if k == 'bin' and e[1] == '*':
            a, b = self.affine(e[2]), self.affine(e[3])
            if a is None or b is None:
                return None
            if not a[1]:
                a, b = b, a
            if b[1]:
                return None
            return a[0] * b[0], {n: c * b[0] for n, c in a[1].items()}
        return None

    def epilogue(self, s, c, fused, env, value, out, ind):
        """Store the contraction's result at the point bound in env, then run
        the fused statements for that point."""
        name, axes = s[1], list(s[2])
        venv = dict(env)
        venv['__acc'] = (value, 'float')
        v, t = self.expr(c.epi, venv, out, ind)
        cur = self.fresh('v')
        out.append(f'{ind}const float {cur} = {self.as_float(v, t)};')
        st_line = self.epi_store(name, axes, env, cur)
        if st_line:
            out.append(f'{ind}{st_line}')
        made = {name: cur}
        for kind, t_, inv in fused:
            if kind == 'let':
                def sub(n, made=made):
                    if n[0] == 'idx' and n[1] in made:
                        return ('name', '__cur_' + n[1])
                    return n
                e2 = rebuild(t_[3], sub)
                fenv = dict(env)
                for m, cv in made.items():
                    fenv['__cur_' + m] = (cv, 'float')
                v2, t2 = self.expr(e2, fenv, out, ind)
                nv = self.fresh('v')
                out.append(f'{ind}const float {nv} = {self.as_float(v2, t2)};')
                st_line = self.epi_store(t_[1], list(t_[2]), env, nv)
                if st_line:
                    out.append(f'{ind}{st_line}')
                made[t_[1]] = nv
            else:
                saved_cap, self.capture = self.capture, None
                self.epilogue_emit(t_, inv, env, made, out, ind)
                self.capture = saved_cap

    def epi_store(self, name, axes, env, cur):
        """The store of an epilogue value at the point bound in env: none when
        only statements of the same epilogue read it; into the block's LDS
        copy when its site writes it out afterwards (``out_stage``)."""
        if name in self.skip_store:
            return None
        os_ = self.out_stage.get(name)
        if os_ is not None:
            base, PPB, reg, pts = os_
            row = self.addr([env[a][0] for a in reg], self.strides(reg)) if reg else '0'
            pt = self.addr([env[a][0] for a in pts], self.strides(pts))
            return f'sh_f[{base} + ({row}) * {PPB} + ({pt}) - (int)blockIdx.x * {PPB}] = {cur};'
        if name in self.chain_local:
            return None                 # the early-load pass over an epilogue: no store to make
        return self.store(name, [env[a][0] for a in axes], cur, 'float')

    def epilogue_emit(self, t_, inv, env, made, out, ind):
        if True:
            if True:
                src, plan = inv
                lines, cond, eenv = [], [], dict(env)
                for axis, const, order, radix in plan:
                    rel = self.fresh('rel')
                    lines.append(f'const int {rel} = {env[axis][0]} - ({const});')
                    cond.append(f'{rel} >= 0 && {rel} < {radix}')
                    rem = rel
                    r2 = radix
                    for a in order:
                        r2 //= self.static[a]
                        lines.append(f'const int i_{a} = ({rem}) / {r2};' if r2 > 1 else f'const int i_{a} = {rem};')
                        if r2 > 1:
                            nr = self.fresh('rm')
                            lines.append(f'const int {nr} = ({rem}) % {r2};')
                            rem = nr
                        eenv[a] = (f'i_{a}', 'int')
                out.append(f'{ind}{{')
                for ln in lines:
                    out.append(f'{ind}  {ln}')
                out.append(f'{ind}  if ({" && ".join(cond)}) {{')
                e2 = replace_node(t_[3], src, ('name', '__cur_' + src[1]))
                for m, cv in made.items():
                    eenv['__cur_' + m] = (cv, 'float')
                inner = []
                ix = [self.index(x, eenv, inner, ind + '    ') for x in t_[2]]
                v2, t2 = self.expr(e2, eenv, inner, ind + '    ')
                out += inner
                out.append(f'{ind}    {self.res_store(t_[1], ix, v2, t2, t_[2])}')
                out.append(f'{ind}  }}')
                out.append(f'{ind}}}')

    def res_store(self, n, ix, v, t, exprs=None):
        dt = self.res[n][1]
        if exprs is not None:
            ix = [self.clamp(i, x, d) for i, x, d in zip(ix, exprs, self.res[n][0])]
        a = self.addr(ix, self.res_strides(n))
        if dt == 'f16':
            return f'stc_h(rb_{n}, {a}, {self.as_float(v, t)});'
        if dt == 'f32':
            return f'stc(R_{n} + {a}, {self.as_float(v, t)});'
        return f'stc_i(R_{n} + {a}, (int)({v}));'

    def site_io(self, s, c, fused):
        exprs = [s[3]]
        writes = {self.root(s[1])}
        for kind, t, _ in fused:
            exprs += stmt_exprs(t)
            writes.add(self.root(t[1]) if kind == 'let' else t[1])
        made = {s[1]} | {t[1] for kind, t, _ in fused if kind == 'let'}
        return self.root_reads(exprs, exclude=made), writes

    def note(self, reads, writes):
        self.dirty |= {n for n in writes if n not in self.private}
        self.trace.append(('note', frozenset(n for n in reads if n not in self.private),
                           frozenset(n for n in writes if n not in self.private)))

    # -- tile
    def gen_tile(self, s, c, fused, out, ind):
        name, axes = s[1], list(s[2])
        reads, writes = self.site_io(s, c, fused)
        self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s), 'tile' + (f' +{len(fused)} fused' if fused else '')))
        for _, t, _ in fused:
            self.plan.append((show_stmt(t), f'epilogue of {name}'))
        dt = self.res[c.W][1]
        vec = c.vec
        J = self.static[c.contig]
        nvec = J // vec
        lpr = 1
        while lpr * 2 <= TILE_LANES and nvec % (lpr * 2) == 0:
            lpr *= 2
        tj = lpr * vec
        nj = J // tj
        rpw = WAVE // lpr
        rpb = rpw * NWAVE
        reg = c.reg_axes
        rn = self.size(reg)
        chunks = [reg[:]]           # register rows are processed in chunks of REG_MAX
        rch = min(rn, REG_MAX)
        nrch = (rn + rch - 1) // rch
        pt = c.pt_axes
        npt_max = self.size(pt)
        nt_max = npt_max * nj * nrch
        poff = self.alloc_scratch(nt_max * KCAP * rch * tj)
        coff = self.alloc_counters(nt_max)
        self.red_floats = max(getattr(self, 'red_floats', 4), NWAVE * rch * tj)
        I = ind + '  '
        o = out
        o.append(f'{ind}{{  // tile {name}: W={c.W} VEC={vec} lanes/row={lpr} cols/tile={tj} reg={rn}')
        o.append(f'{I}const int K_ = {self.count_c(c.fold_axes)};')
        o.append(f'{I}const int NT_ = {self.count_c(pt)} * {nj * nrch};')
        o.append(f'{I}int ks_ = (int)nblk / NT_; ks_ = ks_ < 1 ? 1 : (ks_ > {KCAP} ? {KCAP} : ks_);')
        o.append(f'{I}{{ const int mk_ = (K_ + {rpb - 1}) / {rpb}; if (ks_ > mk_) ks_ = mk_; if (ks_ < 1) ks_ = 1; }}')
        o.append(f'{I}const int rows_ = (K_ + ks_ - 1) / ks_;')
        o.append(f'{I}const int nitem_ = NT_ * ks_;')
        o.append(f'{I}const int sub_ = lane / {lpr}, cl_ = lane % {lpr};')
        o.append(f'{I}for (int it_ = blockIdx.x; it_ < nitem_; it_ += nblk) {{')
        J2 = I + '  '
        o.append(f'{J2}const int c_ = it_ % ks_, tl_ = it_ / ks_;')
        o.append(f'{J2}const int jt_ = tl_ % {nj}; int pq_ = tl_ / {nj};')
        o.append(f'{J2}const int rc_ = pq_ % {nrch}; pq_ /= {nrch};')
        env = self.decode('pq_', pt, o, J2)
        o.append(f'{J2}const int jc_ = jt_ * {tj} + cl_ * {vec};')
        o.append(f'{J2}float acc_[{rch}][{vec}];')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int r_ = 0; r_ < {rch}; ++r_)')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int v_ = 0; v_ < {vec}; ++v_) acc_[r_][v_] = 0.0f;')
        o.append(f'{J2}const int k0_ = c_ * rows_;')
        o.append(f'{J2}const int k1_ = k0_ + rows_ < K_ ? k0_ + rows_ : K_;')
        o.append(f'{J2}const int kb_ = k0_ + wave * {rpw} + sub_;')
        o.append(f'{J2}const int n_ = kb_ < k1_ ? (k1_ - kb_ + {rpb - 1}) / {rpb} : 0;')
        o.append(f'{J2}for (int b_ = 0; b_ < n_; b_ += {UNROLL}) {{')
        K3 = J2 + '  '
        ltype = {8: 'vh_u32x4', 4: 'vh_u32x2', 2: 'unsigned', 1: 'vh_half'}[vec] if dt == 'f16' else \
            {4: 'vh_f32x4', 2: 'vh_f32x2', 1: 'float'}[vec]
        o.append(f'{K3}{ltype} wq_[{UNROLL}];')
        o.append(f'{K3}float av_[{UNROLL}][{rch}];')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int u_ = 0; u_ < {UNROLL}; ++u_) {{')
        K4 = K3 + '  '
        o.append(f'{K4}if (b_ + u_ < n_) {{')
        K5 = K4 + '  '
        o.append(f'{K5}const int kr_ = kb_ + (b_ + u_) * {rpb};')
        kenv = self.decode('kr_', c.fold_axes, o, K5, prefix='f_')
        wenv = {**env, **kenv, c.contig: ('jc_', 'int')}
        for a in reg:
            wenv[a] = ('0', 'int')
        pre = []
        wix = [self.index(x, wenv, pre, K5) for x in c.widx]
        o += pre
        waddr = self.addr(wix, self.res_strides(c.W))
        o.append(f'{K5}wq_[u_] = {self.vec_load(dt, vec, c.W, waddr)};')
        # the other factor for every register row, read in the same batch as the weights
        for r in range(rch):
            renv = {**env, **kenv}
            if reg:
                rl = []
                renv.update(self.decode_const(f'(rc_ * {rch} + {r})', reg, rl, K5))
                o += rl
            pre = []
            av, at = self.expr(c.A, renv, pre, K5)
            o += pre
            if rn % rch:
                o.append(f'{K5}av_[u_][{r}] = (rc_ * {rch} + {r} < {rn}) ? {self.as_float(av, at)} : 0.0f;')
            else:
                o.append(f'{K5}av_[u_][{r}] = {self.as_float(av, at)};')
        o.append(f'{K4}}} else {{')
        o.append(f'{K5}wq_[u_] = {self.vec_zero(dt, vec)};')
        o.append(f'{K5}#pragma unroll')
        o.append(f'{K5}for (int r_ = 0; r_ < {rch}; ++r_) av_[u_][r_] = 0.0f;')
        o.append(f'{K4}}}')
        o.append(f'{K3}}}')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int u_ = 0; u_ < {UNROLL}; ++u_) {{')
        o.append(f'{K4}float wf_[{vec}];')
        o.append(f'{K4}{self.vec_unpack(dt, vec, "wq_[u_]", "wf_")}')
        o.append(f'{K4}#pragma unroll')
        o.append(f'{K4}for (int r_ = 0; r_ < {rch}; ++r_)')
        o.append(f'{K4}  #pragma unroll')
        o.append(f'{K4}  for (int v_ = 0; v_ < {vec}; ++v_) acc_[r_][v_] = fmaf(av_[u_][r_], wf_[v_], acc_[r_][v_]);')
        o.append(f'{K3}}}')
        o.append(f'{J2}}}')
        # reduce over rows inside the wave, then across waves through LDS
        if lpr < 64:
            o.append(f'{J2}#pragma unroll')
            o.append(f'{J2}for (int r_ = 0; r_ < {rch}; ++r_)')
            o.append(f'{J2}  #pragma unroll')
            o.append(f'{J2}  for (int v_ = 0; v_ < {vec}; ++v_) acc_[r_][v_] = wave_red_sum_hi(acc_[r_][v_], {lpr});')
        o.append(f'{J2}if (sub_ == 0) {{')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int r_ = 0; r_ < {rch}; ++r_)')
        o.append(f'{J2}    #pragma unroll')
        o.append(f'{J2}    for (int v_ = 0; v_ < {vec}; ++v_) red_sh[(wave * {rch} + r_) * {tj} + cl_ * {vec} + v_] = '
                 f'acc_[r_][v_];')
        o.append(f'{J2}}}')
        o.append(f'{J2}vh_lds_sync();')
        q = rch * tj

        def finish(val, lines, ind2):
            lines.append(f'{ind2}const int r_ = q_ / {tj}, col_ = q_ % {tj};')
            fenv = dict(env)
            if reg:
                lines.append(f'{ind2}const int rf_ = rc_ * {rch} + r_;')
                fenv.update(self.decode('rf_', reg, lines, ind2))
                lines.append(f'{ind2}if (rf_ < {rn}) {{')
                ind3 = ind2 + '  '
            else:
                ind3 = ind2
            lines.append(f'{ind3}const int i_{c.contig} = jt_ * {tj} + col_;')
            fenv[c.contig] = (f'i_{c.contig}', 'int')
            self.epilogue(s, c, fused, fenv, val, lines, ind3)
            if reg:
                lines.append(f'{ind2}}}')

        o.append(f'{J2}if (ks_ == 1) {{')
        o.append(f'{J2}  for (int q_ = tid; q_ < {q}; q_ += {BLOCK}) {{')
        o.append(f'{J2}    const float s_ = ' + ' + '.join(f'red_sh[{w * q} + q_]' for w in range(NWAVE)) + ';')
        finish('s_', o, J2 + '    ')
        o.append(f'{J2}  }}')
        o.append(f'{J2}}} else {{')
        o.append(f'{J2}  for (int q_ = tid; q_ < {q}; q_ += {BLOCK})')
        o.append(f'{J2}    stc(S + {poff} + (size_t)it_ * {q} + q_, '
                 + ' + '.join(f'red_sh[{w * q} + q_]' for w in range(NWAVE)) + ');')
        o.append(f'{J2}  if (last_arrival(bar + {coff} + tl_ * {LINE_WORDS}, (unsigned)ks_, &flag_sh)) {{')
        o.append(f'{J2}    for (int q_ = tid; q_ < {q}; q_ += {BLOCK}) {{')
        o.append(f'{J2}      float p_[{KCAP}];')
        o.append(f'{J2}      #pragma unroll')
        o.append(f'{J2}      for (int c2_ = 0; c2_ < {KCAP}; ++c2_) '
                 f'p_[c2_] = c2_ < ks_ ? ldc(S + {poff} + (size_t)(tl_ * ks_ + c2_) * {q} + q_) : 0.0f;')
        o.append(f'{J2}      float s_ = p_[0];')
        o.append(f'{J2}      #pragma unroll')
        o.append(f'{J2}      for (int c2_ = 1; c2_ < {KCAP}; ++c2_) if (c2_ < ks_) s_ += p_[c2_];')
        finish('s_', o, J2 + '      ')
        o.append(f'{J2}    }}')
        o.append(f'{J2}  }}')
        o.append(f'{J2}}}')
        o.append(f'{J2}vh_lds_sync();')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')
        self.note(reads, writes)
        self.mark(out, ind, f'tile {name}')

    def decode_const(self, flat, axes, out, ind):
        """Bind axes from a flat index expression (row-major)."""
        v = self.fresh('rr')
        out.append(f'{ind}const int {v} = {flat};')
        return self.decode(v, axes, out, ind, prefix=self.fresh('g') + '_')

    def vec_load(self, dt, vec, W, addr):
        if self.coherent(W):
            if dt == 'f16' and vec == 8:
                return f'ldc16_h(rb_{W}, {addr})'
            if dt == 'f16' and vec == 4:
                return f'ldc8_h(rb_{W}, {addr})'
            raise LowerError(f'coherent load of {W}: vector width {vec} ({dt}) not supported')
        if dt == 'f16':
            if vec == 8:
                return f'ld16_nt(R_{W} + {addr})'
            if vec == 4:
                return f'ld8_nt(R_{W} + {addr})'
            if vec == 2:
                return f'*(const unsigned*)(R_{W} + {addr})'
            return f'R_{W}[{addr}]'
        if vec == 4:
            return f'__builtin_nontemporal_load((const vh_f32x4*)(R_{W} + {addr}))'
        if vec == 2:
            return f'*(const vh_f32x2*)(R_{W} + {addr})'
        return f'R_{W}[{addr}]'

    def vec_zero(self, dt, vec):
        if dt == 'f16':
            return {8: 'vh_u32x4{0u, 0u, 0u, 0u}', 4: 'vh_u32x2{0u, 0u}', 2: '0u', 1: '(vh_half)0'}[vec]
        return {4: 'vh_f32x4{0.f, 0.f, 0.f, 0.f}', 2: 'vh_f32x2{0.f, 0.f}', 1: '0.0f'}[vec]

    def vec_unpack(self, dt, vec, src, dst):
        if dt == 'f16':
            if vec == 8:
                return f'unpack8({src}, {dst});'
            if vec == 4:
                return f'unpack4({src}, {dst});'
            if vec == 2:
                return f'{dst}[0] = h2f_lo({src}); {dst}[1] = h2f_hi({src});'
            return f'{dst}[0] = h2f({src});'
        if vec == 4:
            return f'{dst}[0] = {src}.x; {dst}[1] = {src}.y; {dst}[2] = {src}.z; {dst}[3] = {src}.w;'
        if vec == 2:
            return f'{dst}[0] = {src}.x; {dst}[1] = {src}.y;'
        return f'{dst}[0] = {src};'

    # -- lane
    def gen_lane(self, s, c, fused, out, ind):
        name = s[1]
        reads, writes = self.site_io(s, c, fused)
        self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s), 'lane' + (f' +{len(fused)} fused' if fused else '')))
        for _, t, _ in fused:
            self.plan.append((show_stmt(t), f'epilogue of {name}'))
        self.emit_lane(s, c, fused, out, ind, c.pt_axes, {}, 'blockIdx.x * %d + wave' % NWAVE, f'nblk * {NWAVE}')
        self.note(reads, writes)
        self.mark(out, ind, f'lane {name}')

    def emit_lane(self, s, c, fused, out, ind, pt, base_env, wave_c, nwave_c):
        """A group of lanes per output point, 16-byte loads along the fold.
        Each wave takes PI points per lane group at once (PI x per-lane loads
        in flight); when the other factor does not depend on the point (the
        LM head's c[bt, d]) each lane keeps its slice of it in registers.
        Points are the axes ``pt`` (others come bound in ``base_env``), taken
        by waves ``wave_c`` of ``nwave_c``."""
        name = s[1]
        dt = self.res[c.W][1]
        vec = c.vec
        K = self.static[c.contig]
        nv = K // vec
        reg = c.reg_axes
        rn = self.size(reg)
        rch = min(rn, REG_MAX)
        nrch = (rn + rch - 1) // rch
        preload = nrch == 1 and (self.free_axes(c.A) - {c.contig}) <= set(reg) | set(base_env)
        lpp = 1
        while lpp * 2 <= 64 and nv % (lpp * 2) == 0:
            lpp *= 2
        if lpp < 8 and nv >= 64:
            lpp = 64
        if preload and -(-nv // lpp) * vec * rch > 128 and nv >= 64:
            lpp = 64
        pl = -(-nv // lpp)                       # vectors per lane
        exact = nv % lpp == 0
        ppw = WAVE // lpp
        PI = max(1, min(8, 12 // pl, 32 // rch))
        step = ppw * PI
        I = ind + '  '
        o = out
        ltype = {8: 'vh_u32x4', 4: 'vh_u32x2', 2: 'unsigned', 1: 'vh_half'}[vec] if dt == 'f16' else \
            {4: 'vh_f32x4', 2: 'vh_f32x2', 1: 'float'}[vec]
        o.append(f'{ind}{{  // lane {name}: W={c.W} VEC={vec} lanes/point={lpp} points/iter={PI} reg={rn}'
                 f'{" preloaded" if preload else ""}')
        o.append(f'{I}const int NP_ = {self.count_c(pt)} * {nrch};')
        o.append(f'{I}const int sub_ = lane / {lpp}, cl_ = lane % {lpp};')
        o.append(f'{I}const int gw_ = {wave_c}, nw_ = {nwave_c};')
        kcond = '' if exact else f' && kv_ < {K}'
        if preload:
            o.append(f'{I}float ap_[{pl}][{vec}][{rch}];')
            o.append(f'{I}#pragma unroll')
            o.append(f'{I}for (int m_ = 0; m_ < {pl}; ++m_) {{')
            o.append(f'{I}  const int kv_ = (cl_ + m_ * {lpp}) * {vec};')
            o.append(f'{I}  #pragma unroll')
            o.append(f'{I}  for (int v_ = 0; v_ < {vec}; ++v_) {{')
            o.append(f'{I}    const int kk_ = kv_ + v_;')
            for r in range(rch):
                renv = {**base_env, c.contig: ('kk_', 'int')}
                if reg:
                    rl = []
                    renv.update(self.decode_const(str(r), reg, rl, I + '    '))
                    o += rl
                pre = []
                av, at = self.expr(c.A, renv, pre, I + '    ')
                o += pre
                o.append(f'{I}    ap_[m_][v_][{r}] = {"" if exact else f"kk_ >= {K} ? 0.0f : "}{self.as_float(av, at)};')
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        o.append(f'{I}for (int p0_ = gw_ * {step}; p0_ < NP_; p0_ += nw_ * {step}) {{')
        J2 = I + '  '
        o.append(f'{J2}bool ok_[{PI}];')
        o.append(f'{J2}int prc_[{PI}];')
        for a in pt:
            o.append(f'{J2}int px_{a}[{PI}];')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int pi_ = 0; pi_ < {PI}; ++pi_) {{')
        o.append(f'{J2}  const int p_ = p0_ + pi_ * {ppw} + sub_;')
        o.append(f'{J2}  ok_[pi_] = p_ < NP_;')
        o.append(f'{J2}  int pq_ = ok_[pi_] ? p_ : 0;')
        o.append(f'{J2}  prc_[pi_] = pq_ % {nrch}; pq_ /= {nrch};')
        for a in reversed(pt[1:]):
            o.append(f'{J2}  px_{a}[pi_] = pq_ % {self.ext_c(a)}; pq_ /= {self.ext_c(a)};')
        if pt:
            o.append(f'{J2}  px_{pt[0]}[pi_] = pq_;')
        o.append(f'{J2}}}')
        env = {**base_env, **{a: (f'px_{a}[pi_]', 'int') for a in pt}}
        o.append(f'{J2}{ltype} wq_[{PI}][{pl}];')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int pi_ = 0; pi_ < {PI}; ++pi_)')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int m_ = 0; m_ < {pl}; ++m_) {{')
        K4 = J2 + '    '
        o.append(f'{K4}const int kv_ = (cl_ + m_ * {lpp}) * {vec};')
        o.append(f'{K4}if (ok_[pi_]{kcond}) {{')
        wenv = {**env, c.contig: ('kv_', 'int')}
        for a in reg:
            wenv[a] = ('0', 'int')
        pre = []
        wix = [self.index(x, wenv, pre, K4 + '  ') for x in c.widx]
        o += pre
        waddr = self.addr(wix, self.res_strides(c.W))
        o.append(f'{K4}  wq_[pi_][m_] = {self.vec_load(dt, vec, c.W, waddr)};')
        o.append(f'{K4}}} else {{')
        o.append(f'{K4}  wq_[pi_][m_] = {self.vec_zero(dt, vec)};')
        o.append(f'{K4}}}')
        o.append(f'{J2}  }}')
        o.append(f'{J2}float acc_[{PI}][{rch}];')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int pi_ = 0; pi_ < {PI}; ++pi_) {{')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int r_ = 0; r_ < {rch}; ++r_) acc_[pi_][r_] = 0.0f;')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int m_ = 0; m_ < {pl}; ++m_) {{')
        K5 = J2 + '    '
        o.append(f'{K5}const int kv_ = (cl_ + m_ * {lpp}) * {vec};')
        o.append(f'{K5}float wf_[{vec}];')
        o.append(f'{K5}{self.vec_unpack(dt, vec, "wq_[pi_][m_]", "wf_")}')
        o.append(f'{K5}#pragma unroll')
        o.append(f'{K5}for (int v_ = 0; v_ < {vec}; ++v_) {{')
        K6 = K5 + '  '
        o.append(f'{K6}const int kk_ = kv_ + v_;')
        for r in range(rch):
            if preload:
                o.append(f'{K6}acc_[pi_][{r}] = fmaf(ap_[m_][v_][{r}], wf_[v_], acc_[pi_][{r}]);')
                continue
            renv = {**env, c.contig: ('kk_', 'int')}
            if reg:
                rl = []
                renv.update(self.decode_const(f'(prc_[pi_] * {rch} + {r})', reg, rl, K6))
                o += rl
            pre = []
            av, at = self.expr(c.A, renv, pre, K6)
            o += pre
            guards = []
            if rn % rch:
                guards.append(f'prc_[pi_] * {rch} + {r} < {rn}')
            if not exact:
                guards.append(f'kk_ < {K}')
            g = ' && '.join(guards)
            if g:
                o.append(f'{K6}if ({g}) acc_[pi_][{r}] = fmaf({self.as_float(av, at)}, wf_[v_], acc_[pi_][{r}]);')
            else:
                o.append(f'{K6}acc_[pi_][{r}] = fmaf({self.as_float(av, at)}, wf_[v_], acc_[pi_][{r}]);')
        o.append(f'{K5}}}')
        o.append(f'{J2}  }}')
        o.append(f'{J2}}}')
        if lpp > 1:
            o.append(f'{J2}#pragma unroll')
            o.append(f'{J2}for (int pi_ = 0; pi_ < {PI}; ++pi_)')
            o.append(f'{J2}  #pragma unroll')
            o.append(f'{J2}  for (int r_ = 0; r_ < {rch}; ++r_) acc_[pi_][r_] = group_red_sum(acc_[pi_][r_], {lpp});')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int pi_ = 0; pi_ < {PI}; ++pi_) {{')
        o.append(f'{J2}  if (ok_[pi_] && cl_ == 0) {{')
        K3 = J2 + '    '
        for r in range(rch):
            fenv = dict(env)
            lines = []
            if reg:
                lines.append(f'{K3}if (prc_[pi_] * {rch} + {r} < {rn}) {{')
                K4 = K3 + '  '
                fenv.update(self.decode_const(f'(prc_[pi_] * {rch} + {r})', reg, lines, K4))
            else:
                K4 = K3
            self.epilogue(s, c, fused, fenv, f'acc_[pi_][{r}]', lines, K4)
            if reg:
                lines.append(f'{K3}}}')
            o += lines
        o.append(f'{J2}  }}')
        o.append(f'{J2}}}')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')

    # -- private
    def base_after(self, ss, j):
        """The fixed-point base the next site of this phase will store (an
        attention with its projection, or a stream split over its fold), if
        only contractions and their epilogues come between: (statement for the
        plan or None, target, axes, expression, the site's description)."""
        for t in ss[j:]:
            if id(t) in self.proj:
                pj = self.proj[id(t)]
                return pj['sz'], pj['sz'][1], list(pj['sz'][2]), pj['base'], pj
            if id(t) in self.splits:
                sk = self.splits[id(t)]
                return None, self.root(t[1]), list(t[2]), sk['base'], sk
            if id(t) in self.chains:
                ch = self.chains[id(t)]
                return None, ch['z'], list(t[2]), ch['base'], ch
            if t[0] == 'emit' or (t[0] == 'let' and self.place.get(id(t)) in ('tile', 'lane', 'epilogue')
                                  and id(t) not in self.groups):
                continue
            return None
        return None

    def early_spread_loads(self, axes, e, out, ind):
        """For a loop over ``axes`` spread over the grid (point p_ = block +
        nblk * tid, one per thread): issue the residue loads of e into
        registers at the barrier before, as the stream epilogues do, so the
        loop does not wait for them. Returns the register prefix (the loop
        generates e under a capture with it), or None (loads stay in place:
        more points than the compute waves' threads, no barrier to use, or
        matrix-core rows). Measured, same box: GPT-2 small B=1 208.9 -> 205.4
        us per step; B=8 318.4 -> 319.9 (two more spilled registers), so not
        from MFMA_ROWS_MIN rows."""
        if (self.batch >= MFMA_ROWS_MIN or any(a in self.dynamic for a in axes)
                or self.prefetch_target() is None):
            return None
        N = self.size(axes)
        if N > self.grid * (NWAVE - 1) * WAVE:
            return None
        pfx = f'pb_{self.fresh("b")}_'
        unsafe = self.unsafe_early()
        regs, ok = [], [True]

        def make(step_override):
            saved = self.override_step(step_override)
            try:
                lines = ['{ const int p_ = (int)blockIdx.x + (int)nblk * tid;', f'  if (p_ < {N}) {{']
                env = self.decode('p_', axes, lines, '    ')
                self.capture = {'prefix': pfx, 'loads': [], 'unsafe': unsafe}
                pre = []
                self.expr(e, env, pre, '    ')
                got = self.capture['loads']
                if pre:
                    ok[0] = False
                if step_override is None or step_override[0] == '0':
                    regs.extend((n, k) for n, _, k in got)
                lines += [f'    {n} = {t};' for n, t, _ in got]
                return lines + ['  }', '}'] if got and ok[0] else []
            finally:
                self.capture = None
                self.restore_step(saved)
        self.place_prefetch(make, out, ind)
        if not ok[0] or not regs:
            return None
        seen = set()
        for n, k in regs:
            if n not in seen:
                seen.add(n)
                self.decls.append(f'{self.cap_ctype(k)} {n};')
        return pfx, unsafe

    def spread_value(self, e, env, pre, ind, early):
        """e at a point of a grid-spread loop, its residue loads read from the
        registers ``early_spread_loads`` filled."""
        if early is None:
            return self.expr(e, env, pre, ind)
        self.capture = {'prefix': early[0], 'loads': [], 'unsafe': early[1]}
        try:
            return self.expr(e, env, pre, ind)
        finally:
            self.capture = None

    def emit_base(self, shown, z, axes, base, out, ind, sync):
        """z = base at every point (z a fixed-point sum that a later site adds
        into), spread over all blocks, a few threads each."""
        reads = self.root_reads([base])
        if sync:
            self.sync(reads, {z}, out, ind, f'{z} base')
        self.trace.append(('store', z))
        if shown is not None:
            self.plan.append((show_stmt(shown), 'fixed-point sum: base here, projection adds'))
        early = self.early_spread_loads(axes, base, out, ind)
        I = ind + '  '
        out.append(f'{ind}for (int p_ = (int)blockIdx.x + (int)nblk * tid; p_ < {self.count_c(axes)}; '
                   f'p_ += nthr) {{  // {z} base')
        env = self.decode('p_', axes, out, I)
        pre = []
        v, t = self.spread_value(base, env, pre, I, early)
        out += pre
        out.append(f'{I}{self.store(z, [env[a][0] for a in axes], v, t)}')
        out.append(f'{ind}}}')
        self.note(reads, {z})
        self.mark(out, ind, f'{z} base')

    def gen_private(self, run, out, ind, fx_base=None):
        reads = self.root_reads([t[3] for t in run], exclude={t[1] for t in run})
        self.sync(reads, set(), out, ind, run[0][1])
        out.append(f'{ind}vh_lds_sync();')
        # global values the run reads are staged into LDS once (coherent loads)
        base = off = self.lds_floats
        staged = {}
        for r in sorted(reads):
            if r in self.g and r not in self.private:
                size = self.size(self.axes_of[r])
                if off - base + size <= STAGE_MAX:
                    staged[r] = off
                    fn = 'stage_fx' if r in self.fx else 'stage_ldc4'
                    call = f'{fn}(sh_f + {off}, rb_S, {self.gofs(r) if r in self.fx else self.g[r]}, {size});'
                    if r in self.fx_copies:
                        call = (f'stage_fxc<{self.fx_copies[r]}>(sh_f + {off}, rb_S, {self.gofs(r)}, {size}, '
                                f'{self.fx_copy_stride(r)}u);')
                    if r in self.peel_active:
                        lv, zs = self.peel_active[r]
                        out.append(f'{ind}if ({lv} == 0) {{  // {r} starts as {zs[1]}: made here')
                        # every iteration's loads in flight at once (the token rows are random)
                        out.append(f'{ind}  #pragma unroll')
                        out.append(f'{ind}  for (int e_ = tid; e_ < {size}; e_ += {BLOCK}) {{')
                        env = self.decode('e_', list(zs[2]), out, ind + '    ', prefix='z0_')
                        lv_, val = self.peel_value(r, [env[a][0] for a in zs[2]])
                        out.append(f'{ind}    sh_f[{off} + e_] = {val};')
                        out.append(f'{ind}  }}')
                        out.append(f'{ind}}} else {{')
                        out.append(f'{ind}  {call}  // stage {r}')
                        out.append(f'{ind}}}')
                    else:
                        out.append(f'{ind}{call}  // stage {r}')
                    off += -(-size // 4) * 4
        self.stage_floats = max(self.stage_floats, off - base)
        self.priv_stage_end = off - base
        if staged:
            out.append(f'{ind}vh_lds_sync();')
            self.mark(out, ind, f'stage {",".join(staged)}')
        self.staged = staged
        # which waves wrote each value of the run: 'all' (every wave holds every
        # point), 'wave' (point p in wave p % NWAVE) or 'thread' (any thread);
        # a statement waits for the block only when it may read another wave's writes
        wmap = {}
        self.run_wmap = wmap
        for s in run:
            self.plan.append((show_stmt(s), 'private'))
            name, axes, e = s[1], list(s[2]), s[3]
            npts = self.size(axes)
            o = out
            is_fold = e[0] == 'fold' and npts <= 64 and self.static[e[2]] >= 64
            mine = ('all' if npts == 1 else 'wave') if is_fold else 'thread'
            same = [('name', a) for a in axes]
            need = False
            for n in nodes(e):
                if n[0] in ('idx', 'name') and n[1] in wmap:
                    m = wmap[n[1]]
                    if m == 'thread' or (m[0] == 'wave' and not (mine == 'wave' and m[1] == axes
                                                                  and list(n[2]) == same)):
                        need = True
            if need:
                o.append(f'{ind}vh_lds_sync();')
            wmap[name] = ('wave', axes) if mine == 'wave' else mine
            if is_fold:
                self.private_fold(name, axes, e, npts, o, ind)
            elif axes and -(-self.static[axes[-1]] // ((NWAVE - 1) * WAVE)) <= 8:
                self.private_points(s, npts, o, ind)
            else:
                T = -(-npts // BLOCK)
                o.append(f'{ind}#pragma unroll' + ('' if T <= 16 else ' 8'))
                o.append(f'{ind}for (int it_ = 0; it_ < {T}; ++it_) {{  // private {name}')
                I = ind + '  '
                o.append(f'{I}const int p_ = tid + it_ * {BLOCK};')
                o.append(f'{I}if (p_ < {npts}) {{')
                I2 = I + '  '
                env = self.decode('p_', axes, o, I2)
                pre = []
                v, t = self.expr(e, env, pre, I2)
                o += pre
                o.append(f'{I2}{self.store(name, [env[a][0] for a in axes], v, t)}')
                o.append(f'{I}}}')
                o.append(f'{ind}}}')
            self.mark(out, ind, f'private {name}')
        if fx_base is not None:
            # the next site's fixed-point base, from the values staged here
            # (early in the phase, so its loads and stores are not on the path
            # to the phase's end), when nothing read or wrote its target since
            # the last barrier
            shown, z, axes, bexpr, info = fx_base
            if (z not in self.readers and z not in self.dirty
                    and not (self.root_reads([bexpr]) & self.dirty)):
                if (info.get('y') is not None and id(info['y']) in self.chains) or info.get('p2p'):
                    self.chain_base(info, out, ind)
                else:
                    self.emit_base(shown, z, axes, bexpr, out, ind, sync=False)
                info['base_done'] = True
        out.append(f'{ind}vh_lds_sync();')
        self.staged = {}
        self.run_wmap = {}          # which waves hold what holds within this run only

    def private_points(self, s, npts, o, ind):
        """An elementwise private statement: the last axis runs over the threads
        (``tid + j * BLOCK``, j unrolled), the leading axes in a loop. Loads
        that depend only on the last axis and on step variables (layer-norm
        gains) may be issued early, at the barrier before, into registers
        shared by all leading points."""
        name, axes, e = s[1], list(s[2]), s[3]
        lead, last = axes[:-1], axes[-1]
        nl = self.static[last]
        NCT = (NWAVE - 1) * WAVE           # compute threads: the polling wave takes no points
        TJ = -(-nl // NCT)
        nlead = self.size(lead)
        sid = self.fresh('p')
        unsafe = self.unsafe_early()
        # leading points made together: all their LDS reads are issued before
        # any of their stores (a store to LDS keeps later reads behind it)
        LG = max(g for g in range(1, min(nlead, PRIV_GROUP) + 1) if nlead % g == 0)
        lead_vars = [f'i_{a}' for a in lead] + ['pl_', 'pg_'] + [f'i{u}_{a}' for u in range(LG) for a in lead]

        def body_env():
            env = {last: (f'i_{last}', 'int')}
            if lead:
                env.update(self.decode('pl_', lead, [], ''))
            return env

        def frame(jl, inner, with_lead):
            lines = [f'{{ const int i_{last} = tid + {jl * NCT};', f'  if (tid < {NCT} && i_{last} < {nl}) {{']
            if with_lead and lead:
                lines.append(f'    for (int pl_ = 0; pl_ < {nlead}; ++pl_) {{')
                lines += ['      ' + x for x in self.decode_lines('pl_', lead)]
                lines += ['      ' + x for x in inner]
                lines.append('    }')
            else:
                lines += ['    ' + x for x in inner]
            return lines + ['  }', '}']

        regs = []

        def make(step_override):
            saved = dict(self.step_env)
            if step_override is not None and self.loops:
                self.step_env[self.loops[-1]['var']] = step_override
            lines = []
            try:
                for jl in range(TJ):
                    self.capture = {'prefix': f'pp_{sid}_{jl}_', 'loads': [], 'unsafe': unsafe, 'dedupe': {},
                                    'forbid': lead_vars}
                    self.expr(e, body_env(), [], '')
                    got = self.capture['loads']
                    self.capture = None
                    if step_override is None or step_override[0] == '0':
                        regs.extend((n, k) for n, _, k in got)
                    if got:
                        lines += frame(jl, [f'{n} = {t};' for n, t, _ in got], False)
            finally:
                self.capture = None
                self.step_env.clear()
                self.step_env.update(saved)
            return lines
        self.place_prefetch(make, o, ind)
        seen = set()
        for n, k in regs:
            if n not in seen:
                seen.add(n)
                self.decls.append(f'{self.cap_ctype(k)} {n};')
        o.append(f'{ind}// private {name}')
        hv = self.hoist_invariants(e, lead, nlead, o, ind)
        for jl in range(TJ):
            self.capture = {'prefix': f'pp_{sid}_{jl}_', 'loads': [], 'unsafe': unsafe, 'dedupe': {},
                            'forbid': lead_vars}
            try:
                decl, loads, comp = [], [], []
                for u in range(LG):
                    pl = f'(pg_ + {u})' if lead else '0'
                    env = {last: (f'i_{last}', 'int')}
                    if lead:
                        env.update(self.decode(pl, lead, decl, '', prefix=f'i{u}_'))
                    self.lcap = {'prefix': f'lv{u}_', 'loads': [], 'dedupe': {}}
                    self.bind_invariants(hv, pl)
                    pre = []
                    v, t = self.expr(e, env, pre, '')
                    loads += [f'const float {n} = {x};' for n, x in self.lcap['loads']]
                    self.lcap = None
                    comp += pre + [self.store(name, [env[a][0] for a in axes], v, t)]
                inner = decl + loads + comp
                if lead and LG < nlead:
                    inner = ([f'for (int pg_ = 0; pg_ < {nlead}; pg_ += {LG}) {{']
                             + ['  ' + x for x in inner] + ['}'])
                elif lead:
                    inner = ['{ const int pg_ = 0;'] + ['  ' + x for x in inner] + ['}']
                o += [ind + x for x in frame(jl, inner, False)]
            finally:
                self.capture = None
                self.lcap = None
        self.invs, self.divr = {}, {}

    def lead_invariants(self, e, lead):
        """Subexpressions of e (outside folds) that depend on no axis but the
        leading ones (and step variables) and cost a call or a division:
        [(node, is a divisor)], each once."""
        allowed = set(lead) | self.steps
        found, seen = [], set()

        def inv(n):
            return (n[0] != 'num' and self.free_axes(n) <= allowed
                    and not any(x[0] == 'fold' for x in nodes(n)))

        def walk(n):
            if not is_node(n) or n[0] == 'fold':
                return
            if n[0] == 'bin' and n[1] == '/' and n[3][0] != 'num' and inv(n[3]):
                if show(n[3]) not in seen:
                    seen.add(show(n[3]))
                    found.append((n[3], True))
                walk(n[2])
                return
            if n[0] == 'call' and inv(n):
                if show(n) not in seen:
                    seen.add(show(n))
                    found.append((n, False))
                return
            for x in n[1:]:
                for y in (x if isinstance(x, list) else [x]):
                    walk(y)
        walk(e)
        return found

    def hoist_invariants(self, e, lead, nlead, o, ind):
        """Values of e's lead-invariant calls and divisors, once per leading
        point (thread p makes point p) into LDS: [(node, LDS offset, offset of
        the reciprocal or None)]; ``bind_invariants`` then makes the code for
        e's points read them, and divide by such a divisor through its
        reciprocal with the exact residual step. Over one leading point whose
        inputs every wave holds, each thread makes them in registers instead:
        [(node, register, reciprocal register or None, True)]."""
        invs = self.lead_invariants(e, lead) if nlead <= self.BLOCK else []
        if not invs:
            return []
        held = getattr(self, 'run_wmap', {})
        if HOIST_IN_REGISTERS and nlead == 1 and all(
                held.get(n[1]) == 'all' for node, _ in invs for n in nodes(node)
                if n[0] in ('name', 'idx') and self.is_value(n[1])):
            # every wave holds what they read (folds into one point): each
            # thread makes the values itself, the same operations in the same order
            sid = self.fresh('hv')
            env = self.decode('0', lead, o, ind, prefix=f'{sid}_')
            hv = []
            for k, (node, is_div) in enumerate(invs):
                pre = []
                v, t = self.expr(node, env, pre, ind)
                o += pre
                o.append(f'{ind}const float {sid}_{k} = {self.as_float(v, t)};')
                if is_div:
                    o.append(f'{ind}const float {sid}_{k}r = 1.0f / {sid}_{k};')
                hv.append((node, f'{sid}_{k}', f'{sid}_{k}r' if is_div else None, True))
            return hv
        base = self.lds_floats + self.priv_stage_end
        I = ind + '  '
        o.append(f'{ind}if (tid < {nlead}) {{  // once per leading point')
        env = self.decode('tid', lead, o, I, prefix='ip_')
        k, hv = 0, []
        for node, is_div in invs:
            pre = []
            v, t = self.expr(node, env, pre, I)
            o += pre
            o.append(f'{I}{{ const float iv_ = {self.as_float(v, t)};')
            o.append(f'{I}  sh_f[{base + k * nlead} + tid] = iv_;')
            if is_div:
                o.append(f'{I}  sh_f[{base + (k + 1) * nlead} + tid] = 1.0f / iv_;')
                hv.append((node, base + k * nlead, base + (k + 1) * nlead))
                k += 2
            else:
                hv.append((node, base + k * nlead, None))
                k += 1
            o.append(f'{I}}}')
        o.append(f'{ind}}}')
        o.append(f'{ind}vh_lds_sync();')
        self.stage_floats = max(self.stage_floats, self.priv_stage_end + k * nlead)
        return hv

    def bind_invariants(self, hv, pl):
        """The hoisted values of leading point ``pl`` (a C expression)."""
        self.invs, self.divr = {}, {}
        for node, off, roff, *reg in hv:
            if reg:             # made in this thread's registers
                if roff is None:
                    self.invs[show(node)] = off
                else:
                    self.divr[show(node)] = (off, roff)
                continue
            val = self.lds_read(f'sh_f[{off} + {pl}]')
            if roff is None:
                self.invs[show(node)] = val
            else:
                self.divr[show(node)] = (val, self.lds_read(f'sh_f[{roff} + {pl}]'))

    def lds_read(self, text):
        """An LDS read; while ``self.lcap`` collects them, a register it names
        (loaded before the statements that use it)."""
        cap = self.lcap
        if cap is None:
            return text
        got = cap['dedupe'].get(text)
        if got is None:
            got = f"{cap['prefix']}{len(cap['loads'])}"
            cap['loads'].append((got, text))
            cap['dedupe'][text] = got
        return got

    @staticmethod
    def cap_ctype(kind):
        return {'int': 'int', 'float': 'float'}.get(kind, kind)

    def decode_lines(self, var, axes):
        lines = []
        self.decode(var, axes, lines, '')
        return lines

    def private_fold(self, name, axes, e, npts, o, ind):
        """A fold into a few points: a single point is folded by every wave
        (each wave ends holding it, so readers need no block barrier); several
        points go one per wave (point p in wave p % NWAVE), lanes strided
        along the fold, wave butterfly."""
        op, ax, body = e[1], e[2], e[3]
        K = self.static[ax]
        T = -(-K // WAVE)
        first = 'wave' if npts > 1 else '0'
        o.append(f'{ind}for (int p_ = {first}; p_ < {npts}; p_ += {NWAVE if npts > 1 else 1}) {{  // private {name}')
        I = ind + '  '
        env = self.decode('p_', axes, o, I)
        o.append(f'{I}float a_ = {FOLD_INIT[op]};')
        full = K // WAVE if ax not in self.dynamic else 0
        if 0 < full <= 16:
            # whole rounds unrolled here with every LDS read issued before the sums
            loads, comp = [], []
            self.in_fold = True
            try:
                for it in range(full):
                    self.lcap = {'prefix': f'lf{it}_', 'loads': [], 'dedupe': {}}
                    pre = []
                    v, t = self.expr(body, {**env, ax: (f'(lane + {it * WAVE})', 'int')}, pre, I)
                    loads += [f'{I}const float {n} = {x};' for n, x in self.lcap['loads']]
                    self.lcap = None
                    comp += pre + [f'{I}a_ = {FOLD_OP[op]}(a_, {self.as_float(v, t)});']
            finally:
                self.in_fold = False
                self.lcap = None
            o += loads + comp
        if full * WAVE < K or not 0 < full <= 16:
            start = full if 0 < full <= 16 else 0
            o.append(f'{I}#pragma unroll' + ('' if T <= 16 else ' 8'))
            o.append(f'{I}for (int it_ = {start}; it_ < {T}; ++it_) {{')
            o.append(f'{I}  const int k_ = lane + it_ * {WAVE};')
            o.append(f'{I}  if (k_ < {self.ext_c(ax)}) {{')
            pre = []
            self.in_fold = True
            try:
                v, t = self.expr(body, {**env, ax: ('k_', 'int')}, pre, I + '    ')
            finally:
                self.in_fold = False
            o += pre
            o.append(f'{I}    a_ = {FOLD_OP[op]}(a_, {self.as_float(v, t)});')
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        o.append(f'{I}a_ = wave_red_{op}(a_);')
        o.append(f'{I}if (lane == 0) {self.store(name, [env[a][0] for a in axes], "a_", "float")}')
        o.append(f'{ind}}}')

    # -- group
    def gen_group(self, lead, members, out, ind):
        names = {t[1] for t in members}
        local = self.group_local.get(id(members[0]), [])
        reads = self.root_reads([t[3] for t in members], exclude=names)
        writes = {self.root(t[1]) for t in members if t[1] not in local}
        self.sync(reads, writes, out, ind, members[0][1])
        for t in members:
            kind = self.contraction(t)
            self.plan.append((show_stmt(t), f'group[{", ".join(lead)}]' + (f' {kind.kind}' if kind else '')
                              + (' (LDS)' if t[1] in local else '')))
        # values read only inside the group live in LDS, one leading point at a time
        off = self.lds_floats
        self.glocal = {}
        for n in local:
            self.glocal[n] = (off, len(lead))
            off += max(1, self.size(self.axes_of[n][len(lead):]))
        self.stage_floats = max(self.stage_floats, off - self.lds_floats)
        o = out
        I = ind + '  '
        o.append(f'{ind}for (int gp_ = blockIdx.x; gp_ < {self.count_c(lead)}; gp_ += nblk) {{  // group')
        env = self.decode('gp_', lead, o, I)
        for t in members:
            name, axes, e = t[1], list(t[2]), t[3]
            rest = axes[len(lead):]
            c = self.contraction(t)
            if c is not None and self.block_contraction_ok(c, t, len(lead)):
                if c.kind == 'lane':
                    self.emit_lane(t, c, [], o, I, rest, env, 'wave', str(NWAVE))
                else:
                    self.emit_group_tile(t, c, env, o, I)
            elif not rest and e[0] == 'fold':
                op, ax, body = e[1], e[2], e[3]
                o.append(f'{I}{{  // {name}')
                I2 = I + '  '
                o.append(f'{I2}float a_ = {FOLD_INIT[op]};')
                o.append(f'{I2}for (int k_ = tid; k_ < {self.ext_c(ax)}; k_ += {BLOCK}) {{')
                pre = []
                v, ty = self.expr(body, {**env, ax: ('k_', 'int')}, pre, I2 + '  ')
                o += pre
                o.append(f'{I2}  a_ = {FOLD_OP[op]}(a_, {self.as_float(v, ty)});')
                o.append(f'{I2}}}')
                o.append(f'{I2}a_ = block_red_{op}(a_, red_sh);')
                o.append(f'{I2}if (tid == 0) {self.store(name, [env[a][0] for a in axes], "a_", "float")}')
                o.append(f'{I}}}')
            else:
                o.append(f'{I}#pragma unroll 4')
                o.append(f'{I}for (int q_ = tid; q_ < {self.count_c(rest)}; q_ += {BLOCK}) {{  // {name}')
                I2 = I + '  '
                env2 = {**env, **self.decode('q_', rest, o, I2)}
                pre = []
                v, ty = self.expr(e, env2, pre, I2)
                o += pre
                o.append(f'{I2}{self.store(name, [env2[a][0] for a in axes], v, ty)}')
                o.append(f'{I}}}')
            o.append(f'{I}block_sync();')
        o.append(f'{ind}}}')
        self.glocal = {}
        self.note(reads, writes)
        self.mark(out, ind, f'group {members[0][1]}..{members[-1][1]}')

    def emit_group_tile(self, t, c, env, o, ind):
        """One block computes all of t[lead point, j] = sum over the fold of
        A * W[.., j]: lanes along j (16-byte loads), rows of the fold over the
        block's waves, butterfly + LDS reduction over rows."""
        name = t[1]
        dt = self.res[c.W][1]
        vec = c.vec
        J = self.static[c.contig]
        nvec = J // vec
        lpr = 1
        while lpr * 2 <= TILE_LANES and nvec % (lpr * 2) == 0:
            lpr *= 2
        tj = lpr * vec
        nj = J // tj
        rpw = WAVE // lpr
        rpb = rpw * NWAVE
        self.red_floats = max(getattr(self, 'red_floats', 4), NWAVE * tj)
        ltype = {8: 'vh_u32x4', 4: 'vh_u32x2', 2: 'unsigned', 1: 'vh_half'}[vec] if dt == 'f16' else \
            {4: 'vh_f32x4', 2: 'vh_f32x2', 1: 'float'}[vec]
        I = ind + '  '
        o.append(f'{ind}{{  // group tile {name}: W={c.W} VEC={vec} lanes/row={lpr}')
        o.append(f'{I}const int K_ = {self.count_c(c.fold_axes)};')
        o.append(f'{I}const int sub_ = lane / {lpr}, cl_ = lane % {lpr};')
        o.append(f'{I}const int kb_ = wave * {rpw} + sub_;')
        o.append(f'{I}const int n_ = kb_ < K_ ? (K_ - kb_ + {rpb - 1}) / {rpb} : 0;')
        o.append(f'{I}for (int jt_ = 0; jt_ < {nj}; ++jt_) {{')
        J2 = I + '  '
        o.append(f'{J2}const int jc_ = jt_ * {tj} + cl_ * {vec};')
        o.append(f'{J2}float acc_[{vec}];')
        o.append(f'{J2}#pragma unroll')
        o.append(f'{J2}for (int v_ = 0; v_ < {vec}; ++v_) acc_[v_] = 0.0f;')
        o.append(f'{J2}for (int b_ = 0; b_ < n_; b_ += {UNROLL}) {{')
        K3 = J2 + '  '
        o.append(f'{K3}{ltype} wq_[{UNROLL}];')
        o.append(f'{K3}float av_[{UNROLL}];')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int u_ = 0; u_ < {UNROLL}; ++u_) {{')
        K4 = K3 + '  '
        o.append(f'{K4}if (b_ + u_ < n_) {{')
        K5 = K4 + '  '
        o.append(f'{K5}const int kr_ = kb_ + (b_ + u_) * {rpb};')
        kenv = self.decode('kr_', c.fold_axes, o, K5, prefix='f_')
        wenv = {**env, **kenv, c.contig: ('jc_', 'int')}
        pre = []
        wix = [self.index(x, wenv, pre, K5) for x in c.widx]
        o += pre
        o.append(f'{K5}wq_[u_] = {self.vec_load(dt, vec, c.W, self.addr(wix, self.res_strides(c.W)))};')
        pre = []
        av, at = self.expr(c.A, {**env, **kenv}, pre, K5)
        o += pre
        o.append(f'{K5}av_[u_] = {self.as_float(av, at)};')
        o.append(f'{K4}}} else {{')
        o.append(f'{K5}wq_[u_] = {self.vec_zero(dt, vec)};')
        o.append(f'{K5}av_[u_] = 0.0f;')
        o.append(f'{K4}}}')
        o.append(f'{K3}}}')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int u_ = 0; u_ < {UNROLL}; ++u_) {{')
        o.append(f'{K4}float wf_[{vec}];')
        o.append(f'{K4}{self.vec_unpack(dt, vec, "wq_[u_]", "wf_")}')
        o.append(f'{K4}#pragma unroll')
        o.append(f'{K4}for (int v_ = 0; v_ < {vec}; ++v_) acc_[v_] = fmaf(av_[u_], wf_[v_], acc_[v_]);')
        o.append(f'{K3}}}')
        o.append(f'{J2}}}')
        if lpr < 64:
            o.append(f'{J2}#pragma unroll')
            o.append(f'{J2}for (int v_ = 0; v_ < {vec}; ++v_) acc_[v_] = wave_red_sum_hi(acc_[v_], {lpr});')
        o.append(f'{J2}if (sub_ == 0) {{')
        o.append(f'{J2}  #pragma unroll')
        o.append(f'{J2}  for (int v_ = 0; v_ < {vec}; ++v_) red_sh[wave * {tj} + cl_ * {vec} + v_] = acc_[v_];')
        o.append(f'{J2}}}')
        o.append(f'{J2}vh_lds_sync();')
        o.append(f'{J2}if (tid < {tj}) {{')
        K3 = J2 + '  '
        o.append(f'{K3}const float s_ = ' + ' + '.join(f'red_sh[{w * tj} + tid]' for w in range(NWAVE)) + ';')
        o.append(f'{K3}const int i_{c.contig} = jt_ * {tj} + tid;')
        fenv = {**env, c.contig: (f'i_{c.contig}', 'int')}
        venv = dict(fenv)
        venv['__acc'] = ('s_', 'float')
        pre = []
        v, ty = self.expr(c.epi, venv, pre, K3)
        o += pre
        o.append(f'{K3}{self.store(name, [fenv[a][0] for a in t[2]], v, ty)}')
        o.append(f'{J2}}}')
        o.append(f'{J2}vh_lds_sync();')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')

    # -- grid reduction
    def gen_gridred(self, s, out, ind):
        name, axes, e = s[1], list(s[2]), s[3]
        reads = self.root_reads([e])
        writes = {self.root(name)}
        self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s), 'gridred'))
        op, ax, body = e[1], e[2], e[3]
        npts = self.size(axes)
        poff = self.alloc_scratch(npts * GRID_MAX)
        coff = self.alloc_counters(1)
        o = out
        I = ind + '  '
        o.append(f'{ind}{{  // gridred {name}')
        for p in range(npts):
            env = {}
            lines = []
            if axes:
                env = self.decode_const(str(p), axes, lines, I)
            o += lines
            o.append(f'{I}{{')
            o.append(f'{I}  float a_ = {FOLD_INIT[op]};')
            o.append(f'{I}  for (int k_ = gtid; k_ < {self.static[ax]}; k_ += nthr) {{')
            pre = []
            v, t = self.expr(body, {**env, ax: ('k_', 'int')}, pre, I + '    ')
            o += pre
            o.append(f'{I}    a_ = {FOLD_OP[op]}(a_, {self.as_float(v, t)});')
            o.append(f'{I}  }}')
            o.append(f'{I}  a_ = block_red_{op}(a_, red_sh);')
            o.append(f'{I}  if (tid == 0) stc(S + {poff + p * GRID_MAX} + blockIdx.x, a_);')
            o.append(f'{I}}}')
        o.append(f'{I}if (last_arrival(bar + {coff}, nblk, &flag_sh)) {{')
        for p in range(npts):
            env = {}
            lines = []
            if axes:
                env = self.decode_const(str(p), axes, lines, I + '  ')
            o += lines
            o.append(f'{I}  {{')
            o.append(f'{I}    float a_ = {FOLD_INIT[op]};')
            o.append(f'{I}    for (int b_ = tid; b_ < (int)nblk; b_ += {BLOCK}) a_ = {FOLD_OP[op]}(a_, '
                     f'ldc(S + {poff + p * GRID_MAX} + b_));')
            o.append(f'{I}    a_ = block_red_{op}(a_, red_sh);')
            o.append(f'{I}    if (tid == 0) {self.store(name, [env[a][0] for a in axes], "a_", "float")}')
            o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')
        self.note(reads, writes)
        self.mark(out, ind, f'gridred {name}')

    def gen_argmax(self, s1, s2, out, ind):
        """best = fold max n: E[n]; next = lowest n with E[n] == best: one pass
        over E keeping (value, index) pairs, ties to the lower index. Each
        block reduces the points it made itself when E is a streamed value
        (no grid barrier before), else a grid-strided share; after one grid
        barrier every block combines the per-block pairs in block order, so
        every block holds the result (kept in LDS for block-local feedback)."""
        name, axes, e = s1[1], list(s1[2]), s1[3]
        ax, body = e[2], e[3]
        reads = self.root_reads([e])
        writes = {self.root(name), self.root(s2[1])}
        part, src = None, None
        if body[0] == 'idx' and body[1] in self.axes_of:
            src = self.root(body[1])
            pp = self.stream_part.get(src)
            if (pp and pp['pts'] == [ax] and pp['reg'] == axes and src in self.dirty
                    and list(body[2]) == [('name', a) for a in axes + [ax]]):
                part = pp
        in_lds = self.stream_lds.get(src) if part else None
        if part:
            self.sync(reads - {src}, writes, out, ind, name)
            self.readers.add(src)
            if in_lds is None:
                out.append(f'{ind}block_sync();  // this block\'s own points of {body[1]}')
        else:
            self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s1), 'argmax' + (' (own points)' if part else ' (grid-strided)')))
        self.plan.append((show_stmt(s2), 'argmax'))
        npts = self.size(axes)
        poff = self.alloc_scratch(2 * npts * GRID_MAX)
        o = out
        I = ind + '  '
        o.append(f'{ind}{{  // argmax {name}, {s2[1]}: per-block pairs')
        if in_lds is not None and npts <= NWAVE:
            # wave p reduces row p of the block's LDS copy: no block-wide steps
            o.append(f'{I}if (wave < {npts}) {{')
            o.append(f'{I}  float bv_ = -INFINITY; int bi_ = 0x7fffffff;')
            o.append(f'{I}  const int k0_ = (int)blockIdx.x * {part["PPB"]};')
            o.append(f'{I}  const int k1_ = k0_ + {part["PPB"]} < {part["P"]} ? k0_ + {part["PPB"]} : {part["P"]};')
            o.append(f'{I}  for (int k_ = k0_ + lane; k_ < k1_; k_ += 64) {{')
            o.append(f'{I}    const float v_ = sh_f[{in_lds[0]} + wave * {in_lds[1]} + k_ - k0_];')
            o.append(f'{I}    if (v_ > bv_ || (v_ == bv_ && k_ < bi_)) {{ bv_ = v_; bi_ = k_; }}')
            o.append(f'{I}  }}')
            o.append(f'{I}  wave_argmax(bv_, bi_);')
            o.append(f'{I}  if (lane == 0) {{ stcs(rb_S, {poff} + wave * {GRID_MAX} + blockIdx.x, bv_); '
                     f'stcs(rb_S, {poff + npts * GRID_MAX} + wave * {GRID_MAX} + blockIdx.x, (float)bi_); }}')
            o.append(f'{I}}}')
        envs = []
        for p in (range(npts) if in_lds is None or npts > NWAVE else ()):
            lines = []
            env = self.decode_const(str(p), axes, lines, I) if axes else {}
            envs.append(env)
            o += lines
            o.append(f'{I}{{')
            o.append(f'{I}  float bv_ = -INFINITY; int bi_ = 0x7fffffff;')
            if part:
                o.append(f'{I}  const int k0_ = (int)blockIdx.x * {part["PPB"]};')
                o.append(f'{I}  const int k1_ = k0_ + {part["PPB"]} < {part["P"]} ? k0_ + {part["PPB"]} : {part["P"]};')
                o.append(f'{I}  for (int k_ = k0_ + tid; k_ < k1_; k_ += {BLOCK}) {{')
            else:
                o.append(f'{I}  for (int k_ = gtid; k_ < {self.static[ax]}; k_ += nthr) {{')
            pre = []
            if in_lds is not None:
                # the block's copy in LDS, laid out [row][own point]
                v, t = f'sh_f[{in_lds[0]} + {p * in_lds[1]} + k_ - k0_]', 'float'
            else:
                v, t = self.expr(body, {**env, ax: ('k_', 'int')}, pre, I + '    ')
            o += pre
            o.append(f'{I}    const float v_ = {self.as_float(v, t)};')
            o.append(f'{I}    if (v_ > bv_ || (v_ == bv_ && k_ < bi_)) {{ bv_ = v_; bi_ = k_; }}')
            o.append(f'{I}  }}')
            o.append(f'{I}  block_argmax(bv_, bi_, red_sh, (int*)(red_sh + {NWAVE}));')
            o.append(f'{I}  if (tid == 0) {{ stcs(rb_S, {poff + p * GRID_MAX} + blockIdx.x, bv_); '
                     f'stcs(rb_S, {poff + (npts + p) * GRID_MAX} + blockIdx.x, (float)bi_); }}')
            o.append(f'{I}}}')
        o.append(f'{ind}}}')
        self.barrier(out, ind, f'combine {name}')
        cval = s2[3][3][3][1]
        o.append(f'{ind}{{  // argmax {name}, {s2[1]}: every block combines the pairs in block order')
        if npts <= NWAVE:
            # wave p combines row p
            o.append(f'{I}if (wave < {npts}) {{')
            o.append(f'{I}  float bv_ = -INFINITY; int bi_ = 0x7fffffff;')
            o.append(f'{I}  for (int b_ = lane; b_ < (int)nblk; b_ += 64) {{')
            o.append(f'{I}    const float v_ = ldcs(rb_S, {poff} + wave * {GRID_MAX} + b_);')
            o.append(f'{I}    const int i_ = (int)ldcs(rb_S, {poff + npts * GRID_MAX} + wave * {GRID_MAX} + b_);')
            o.append(f'{I}    if (v_ > bv_ || (v_ == bv_ && i_ < bi_)) {{ bv_ = v_; bi_ = i_; }}')
            o.append(f'{I}  }}')
            o.append(f'{I}  wave_argmax(bv_, bi_);')
            o.append(f'{I}  const float nv_ = bi_ == 0x7fffffff ? {c_float(cval)} : (float)bi_;')
            o.append(f'{I}  if (lane == 0) {{')
            o.append(f'{I}    amx_[wave] = nv_;')
            o.append(f'{I}    if (blockIdx.x == 0) {{')
            env = self.decode('wave', axes, o, I + '      ', prefix='aw_') if axes else {}
            o.append(f'{I}      {self.store(name, [env[a][0] for a in axes], "bv_", "float")}')
            o.append(f'{I}      {self.store(s2[1], [env[a][0] for a in axes], "nv_", "float")}')
            o.append(f'{I}    }}')
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        for p in (range(npts) if npts > NWAVE else ()):
            lines = []
            env = self.decode_const(str(p), axes, lines, I) if axes else {}
            o += lines
            o.append(f'{I}{{')
            o.append(f'{I}  float bv_ = -INFINITY; int bi_ = 0x7fffffff;')
            o.append(f'{I}  for (int b_ = tid; b_ < (int)nblk; b_ += {BLOCK}) {{')
            o.append(f'{I}    const float v_ = ldcs(rb_S, {poff + p * GRID_MAX} + b_);')
            o.append(f'{I}    const int i_ = (int)ldcs(rb_S, {poff + (npts + p) * GRID_MAX} + b_);')
            o.append(f'{I}    if (v_ > bv_ || (v_ == bv_ && i_ < bi_)) {{ bv_ = v_; bi_ = i_; }}')
            o.append(f'{I}  }}')
            o.append(f'{I}  block_argmax(bv_, bi_, red_sh, (int*)(red_sh + {NWAVE}));')
            o.append(f'{I}  const float nv_ = bi_ == 0x7fffffff ? {c_float(cval)} : (float)bi_;')
            o.append(f'{I}  if (tid == 0) {{')
            o.append(f'{I}    amx_[{p}] = nv_;')
            o.append(f'{I}    if (blockIdx.x == 0) {{')
            o.append(f'{I}      {self.store(name, [env[a][0] for a in axes], "bv_", "float")}')
            o.append(f'{I}      {self.store(s2[1], [env[a][0] for a in axes], "nv_", "float")}')
            o.append(f'{I}    }}')
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{ind}}}')
        self.local_vals[s2[1]] = ('amx_', npts)
        self.shared_decls.append(f'__shared__ float amx_[{npts}];')
        self.note(reads, writes)
        self.red_floats = max(getattr(self, 'red_floats', 4), 2 * NWAVE)
        self.mark(out, ind, f'argmax {name}')

    # -- one thread per point
    def gen_repl(self, s, out, ind):
        """Every block computes every point and stores it (identical values),
        then reads only its own stores: no grid barrier is needed before its
        readers, only the block's own drain."""
        name, axes, e = s[1], list(s[2]), s[3]
        reads = self.root_reads([e])
        writes = {self.root(name)}
        self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s), 'replicated'))
        I = ind + '  '
        out.append(f'{ind}for (int p_ = tid; p_ < {self.count_c(axes)}; p_ += {BLOCK}) {{  // replicated {name}')
        env = self.decode('p_', axes, out, I)
        pre = []
        v, t = self.expr(e, env, pre, I)
        out += pre
        out.append(f'{I}{self.store(name, [env[a][0] for a in axes], v, t)}')
        out.append(f'{ind}}}')
        out.append(f'{ind}block_sync();')
        self.readers |= {n for n in reads if n not in self.private}
        self.mark(out, ind, f'replicated {name}')

    def gen_thread(self, s, out, ind):
        name, axes, e = s[1], list(s[2]), s[3]
        reads = self.root_reads([e])
        writes = {self.root(name)}
        self.sync(reads, writes, out, ind, name)
        self.plan.append((show_stmt(s), 'thread'))
        I = ind + '  '
        out.append(f'{ind}#pragma unroll 4')
        out.append(f'{ind}for (int p_ = gtid; p_ < {self.count_c(axes)}; p_ += nthr) {{  // thread {name}')
        env = self.decode('p_', axes, out, I)
        pre = []
        v, t = self.expr(e, env, pre, I)
        out += pre
        out.append(f'{I}{self.store(name, [env[a][0] for a in axes], v, t)}')
        out.append(f'{ind}}}')
        self.note(reads, writes)
        self.mark(out, ind, f'thread {name}')

    def gen_emit(self, s, out, ind):
        name = s[1]
        ax = set()
        for x in list(s[2]) + [s[3]]:
            ax |= self.free_axes(x)
        axes = [a for a in self.static if a in ax and self.is_axis(a)]
        reads = self.root_reads(stmt_exprs(s))
        self.sync(reads, {name}, out, ind, f'emit {name}')
        self.plan.append((show_stmt(s), 'thread emit'))
        I = ind + '  '
        out.append(f'{ind}#pragma unroll 4')
        out.append(f'{ind}for (int p_ = gtid; p_ < {self.count_c(axes)}; p_ += nthr) {{  // emit {name}')
        env = self.decode('p_', axes, out, I)
        pre = []
        ix = [self.index(x, env, pre, I) for x in s[2]]
        v, t = self.expr(s[3], env, pre, I)
        out += pre
        out.append(f'{I}{self.res_store(name, ix, v, t, s[2])}')
        out.append(f'{ind}}}')
        self.note(reads, {name})
        self.mark(out, ind, f'emit {name}')

    def gen_copy(self, dst, src_e, axes, out, ind, what):
        """dst[axes] = src_e, one thread per point (carry copies)."""
        reads = self.root_reads([src_e])
        writes = {self.root(dst)}
        self.sync(reads, writes, out, ind, what)
        I = ind + '  '
        out.append(f'{ind}for (int p_ = gtid; p_ < {self.count_c(axes)}; p_ += nthr) {{  // {what}')
        env = self.decode('p_', list(axes), out, I)
        pre = []
        v, t = self.expr(src_e, env, pre, I)
        out += pre
        out.append(f'{I}{self.store(dst, [env[a][0] for a in axes], v, t)}')
        out.append(f'{ind}}}')
        self.note(reads, writes)

    def writes_of(self, ss):
        """Storage roots and residues the statements write."""
        out = set()
        for t in ss:
            if t[0] in ('let', 'step'):
                out.add(self.root(t[1]))
            if t[0] == 'emit':
                out.add(t[1])
            if t[0] == 'step':
                out |= self.writes_of(t[6])
        return out

    # -- the layer loop
    def gen_step(self, s, out, ind):
        _, name, axes, var, init, carry, blk = s
        self.plan.append((show_stmt(s), 'step loop'))
        if not (init[0] == 'idx' and self.alias.get(init[1]) == carry):
            self.gen_copy(carry, init, axes, out, ind, f'{carry} <- init')
        if var not in self.static:
            raise LowerError(f'step variable {var} needs an axis declaration')
        if self.dirty:
            self.barrier(out, ind, f'step {name}')
        n = self.static[var]
        lv = f'l_{var}'
        out.append(f'{ind}for (int {lv} = 0; {lv} < {self.ext_c(var)}; ++{lv}) {{  // fold step {var}')
        out.append(f'{ind}  const int tid = vh_opaque(tid_k_), lane = tid & 63, wave = tid >> 6;')
        saved = self.step_env.get(var)
        self.step_env[var] = (lv, 'int')
        pe = self.peels.get(id(s))
        if pe is not None:
            self.plan.append((show_stmt(pe), f'first value of {carry}, made where read'))
            self.peel_active[self.root(carry)] = (lv, pe)
        self.mult *= n
        self.trace.append(('loop', var, n))
        self.loops.append({'id': self.fresh('loop'), 'var': var, 'lv': lv, 'n': self.ext_c(var),
                           'pf_before': self.last_pf, 'body_barrier': False, 'end_prefetch': [],
                           'end_dirty': self.writes_of(blk)})
        body = [b for b in blk if b[0] != 'ret']
        ret = [b for b in blk if b[0] == 'ret'][0][1]
        self.gen(body, out, ind + '  ')
        if not (ret[0] == 'idx' and self.alias.get(ret[1]) == carry):
            self.gen_copy(carry, ret, axes, out, ind + '  ', f'{carry} <- ret')
        lp = self.loops[-1]
        self.peel_active.pop(self.root(carry), None)
        self.barrier(out, ind + '  ', f'next {var}', pre_wait=lp['end_prefetch'])
        self.trace.append(('endloop', var))
        self.loops.pop()
        self.mult //= n
        out.append(f'{ind}}}')
        if saved is None:
            del self.step_env[var]
        else:
            self.step_env[var] = saved

    # ------------------------------------------------------------ the kernel
    def plan_feedback(self, feedback):
        """Feedback every block can keep to itself: a token chosen by an
        argmax every block combines, and a step counter. Then no grid barrier
        is needed between steps for it; block 0 alone writes the residues back
        for the host."""
        self.local_fb = {}
        if not feedback:
            return
        tok_srcs = {t[1] for t in self.argmax.values()}
        plan = {}
        for dst, src in feedback.items():
            if dst not in self.res:
                raise NameError(f'feedback target {dst} not supplied')
            shape, dt = self.res[dst]
            if dt != 'i32' or dst in self.emitted:
                return
            if isinstance(src, int):
                if math.prod(shape) != 1:
                    return
                plan[dst] = ('inc', src)
            elif src in tok_srcs and src in self.axes_of and math.prod(shape) == self.size(self.axes_of[src]):
                plan[dst] = ('tok', src)
            else:
                return
        self.local_fb = plan

    def kernel(self, feedback):
        """Body of one step, the feedback stores, and the history of chosen tokens."""
        self.dirty, self.readers = set(), set()
        self.red_floats = 4
        self.plan_feedback(feedback)
        self.head_io = [set(), set()]
        self.first_barrier = False
        body = []
        ind = '    '
        self.gen(self.stmts, body, ind)
        self.history = None
        self.wrap_barrier = True
        if feedback and self.local_fb:
            for dst, (kind, src) in self.local_fb.items():
                if kind == 'inc':
                    body.append(f'{ind}tlv_{dst} += {src};')
                    body.append(f'{ind}if (blockIdx.x == 0 && tid == 0) stc_i(R_{dst}, tlv_{dst});')
                    continue
                arr, n = self.local_vals[src]
                self.history = n
                body.append(f'{ind}if (tid < {n}) {{  // {dst} <- {src}, in every block')
                body.append(f'{ind}  const int nx_ = (int){arr}[tid];')
                body.append(f'{ind}  if (blockIdx.x == 0 && tok_out != nullptr) tok_out[st_ * {n} + tid] = nx_;')
                body.append(f'{ind}  const int xi_ = (tok_in != nullptr && st_ + 1 < nsteps) ? '
                            f'tok_in[(st_ + 1) * {n} + tid] : nx_;')
                body.append(f'{ind}  xfb_{dst}[tid] = xi_;')
                body.append(f'{ind}  if (blockIdx.x == 0) stc_i(R_{dst} + tid, xi_);')
                body.append(f'{ind}}}')
            body.append(f'{ind}vh_lds_sync();')
            # a barrier between steps only if the next step's first phase touches
            # what this step's last phase wrote or read
            hr, hw = self.head_io
            self.wrap_barrier = bool(hr & self.dirty or hw & (self.readers | self.dirty))
            self.trace.append(('feedback', True, frozenset(self.local_fb)))
        elif feedback:
            self.barrier(body, ind, 'feedback')
            self.trace.append(('feedback', False, frozenset(feedback)))
            for dst, src in feedback.items():
                dt = self.res[dst][1]
                if isinstance(src, int):
                    if dt == 'i32':
                        body.append(f'{ind}if (gtid == 0) stc_i(R_{dst}, ldc_i(R_{dst}) + {src});')
                    elif dt == 'f32':
                        body.append(f'{ind}if (gtid == 0) stc(R_{dst}, ldc(R_{dst}) + {src});')
                    else:
                        raise LowerError(f'feedback into fp16 scalar {dst}')
                    continue
                if src not in self.axes_of:
                    raise NameError(f'feedback source {src} is not a value of the program')
                r = self.root(src)
                if r in self.fx:
                    raise LowerError(f'feedback source {src} is a fixed-point sum')
                n = self.size(self.axes_of[r])
                if math.prod(self.res[dst][0]) != n:
                    raise LowerError(f'feedback {dst} <- {src}: {math.prod(self.res[dst][0])} vs {n} elements')
                v = f'ldc(S + {self.g[r]} + gtid)'
                if dt == 'i32' and self.history is None:
                    # token feedback: recorded in tok_out; tok_in (prefill) overrides the next input
                    self.history = n
                    body.append(f'{ind}if (gtid < {n}) {{')
                    body.append(f'{ind}  const int nx_ = (int){v};')
                    body.append(f'{ind}  if (tok_out != nullptr) tok_out[st_ * {n} + gtid] = nx_;')
                    body.append(f'{ind}  stc_i(R_{dst} + gtid, (tok_in != nullptr && st_ + 1 < nsteps) ? '
                                f'tok_in[(st_ + 1) * {n} + gtid] : nx_);')
                    body.append(f'{ind}}}')
                elif dt == 'i32':
                    body.append(f'{ind}if (gtid < {n}) stc_i(R_{dst} + gtid, (int){v});')
                elif dt == 'f32':
                    body.append(f'{ind}if (gtid < {n}) stc(R_{dst} + gtid, {v});')
                else:
                    body.append(f'{ind}if (gtid < {n}) stc_h(rb_{dst}, gtid, {v});')
        return body


def lower(text, res, axis_max, batch=1, per_token=(), outputs=(), feedback=None, timing=False,
          kernel_name='vesta_step', grid=None, prefetch_vgprs=None, mfma_pipe=None):
    """Program text -> Lowered: HIP source of one persistent kernel.

    Kernel ABI: ``<kernel_name>(R_<residue>... in spec order, float* S,
    unsigned* bar, unsigned long long* TS, int nsteps, int* tok_out,
    const int* tok_in)``. ``timing``: True adds per-site clock sums (TS
    [site][block]) and, after them, each block's arrival and release time at
    the barriers of a launch's last step; 'trace' records only the latter (no
    clock reads between barriers). One launch runs ``nsteps`` steps back to back
    (feedback between them; reference launches always run one). With token
    feedback, the token chosen at step k of the launch is stored in
    ``tok_out[k * B + b]`` when ``tok_out`` is not null, and when ``tok_in``
    is not null the input of step k + 1 is ``tok_in[(k + 1) * B + b]``
    instead (prefill: a prompt in one launch). ``bar`` must be zero before
    the first launch and is left consistent by every launch.
    """
    args = (text, res, axis_max, batch, per_token, outputs, feedback, timing, kernel_name)
    out, low = _lower(*args, grid, prefetch_vgprs, mfma_pipe)
    if low.grid_auto and low.grid != GRID_WIDE and (low.proj_wider or out.shared_bytes > LDS_BYTES):
        # the default grid is too small for replicated attention projections, or leaves streams so
        # many points per block that their staged rows overflow LDS; the full grid may not
        out, low = _lower(*args, GRID_WIDE, prefetch_vgprs, mfma_pipe)
    return out


def _lower(text, res, axis_max, batch, per_token, outputs, feedback, timing, kernel_name, grid, prefetch_vgprs,
           mfma_pipe):
    """One lowering on one grid: (Lowered, the Lowering that made it); again
    without local folds when one cannot be kept."""
    args = (text, res, axis_max, batch, per_token, outputs, feedback, timing, kernel_name, grid, prefetch_vgprs,
            mfma_pipe)
    try:
        return _lower_once(*args, local_folds=True)
    except ChainError:
        return _lower_once(*args, local_folds=False)


def _lower_once(text, res, axis_max, batch, per_token, outputs, feedback, timing, kernel_name, grid,
                prefetch_vgprs, mfma_pipe, local_folds):
    stmts = batch_lift(parse(text), batch, set(per_token))
    low = Lowering(stmts, dict(res), axis_max, outputs, batch, timing, grid, prefetch_vgprs, mfma_pipe,
                   local_folds)
    for o in outputs:
        if o not in low.axes_of:
            raise NameError(f'output {o} is not a value of the program')
        if low.root(o) in low.private:
            raise LowerError(f'output {o} was placed in LDS')
    low.fb_targets = set(feedback or {})
    body = low.kernel(feedback)
    # prefetch code goes where each barrier left room for it
    filled = []
    for line in body:
        t = line.strip()
        if t.startswith('/*@PF') and t.endswith('@*/'):
            slot = low.pf_slots[int(t[5:-3])]
            filled += [slot['ind'] + x for x in slot['lines']]
        elif t.startswith('/*@PZ') and t.endswith('@*/'):
            k = int(t[5:-3])
            if k < len(low.pf_slots):
                slot = low.pf_slots[k]
                filled += [slot['ind'] + x for x in slot['pre']]
        else:
            filled.append(line)
    body = filled
    written = set(low.emitted) | low.fb_targets
    params, args = [], []
    for name, (shape, dt) in low.res.items():
        w = name in written
        params.append((name, dt, w))
        args.append(f'{"" if w else "const "}{CTYPE[dt]}* __restrict__ R_{name}')
    args += ['float* __restrict__ S', 'unsigned* __restrict__ bar', 'unsigned long long* __restrict__ TS',
             'const int nsteps', 'int* __restrict__ tok_out', 'const int* __restrict__ tok_in']
    pre = [f'  const vh_rsrc rb_S = mk_rsrc(S, {max(1, low.goff) * 4}u);']
    for name in sorted(written):
        shape, dt = low.res[name]
        if dt == 'f16':
            nbytes = math.prod(shape) * 2
            if nbytes >= 1 << 32:
                raise LowerError(f'residue {name} is {nbytes} bytes; coherent fp16 access is limited to 4 GiB')
            pre.append(f'  const vh_rsrc rb_{name} = mk_rsrc(R_{name}, {nbytes}u);')
    head = []
    # scalar residues read by name: once per step (before any barrier of the step)
    for name, (shape, dt) in low.res.items():
        if math.prod(shape) == 1 and len(shape) <= 1 and name not in low.emitted:
            cty = {'i32': 'int', 'f32': 'float', 'f16': 'float'}[dt]
            if name in low.local_fb:
                val = f'xfb_{name}[0]' if low.local_fb[name][0] == 'tok' else f'tlv_{name}'
            elif low.coherent(name):
                val = {'i32': f'ldc_i(R_{name})', 'f32': f'ldc(R_{name})', 'f16': f'ldc_h(rb_{name}, 0)'}[dt]
            else:
                val = f'h2f(R_{name}[0])' if dt == 'f16' else f'R_{name}[0]'
            head.append(f'    const {cty} rs_{name} = {val};')
    for a, e in low.dynamic.items():
        lines = []
        v = low.index(e, {}, lines, '    ')
        head += lines
        head.append(f'    const int E_{a} = {v};')
        head.append(f'    if (E_{a} > {low.static[a]} || E_{a} < 1) break;  // beyond its bound: stop')
    # block-local feedback state: the chosen tokens in LDS, step counters in registers
    fb_init = []
    for name, (kind, _) in low.local_fb.items():
        n = math.prod(low.res[name][0])
        if kind == 'tok':
            fb_init += [f'  __shared__ int xfb_{name}[{n}];\n',
                        f'  for (int i_ = tid; i_ < {n}; i_ += {BLOCK}) xfb_{name}[i_] = ldc_i(R_{name} + i_);\n']
        else:
            fb_init.append(f'  int tlv_{name} = ldc_i(R_{name});\n')
    if fb_init:
        fb_init.append('  vh_lds_sync();\n')
    red = max(low.red_floats, 4)
    prelude = PRELUDE_PATH.read_text()
    src = (f'#define VBLOCK {BLOCK}\n' + prelude + '\n'
           + f'extern "C" __global__ void __launch_bounds__({BLOCK}, 1) {kernel_name}(' + ', '.join(args) + ') {\n'
           + '  extern __shared__ __attribute__((aligned(16))) float sh_f[];  // 16-byte vector reads\n'
           + f'  __shared__ float red_sh[{red}];\n'
           + '  __shared__ int flag_sh;\n'
           + '  const int tid_k_ = threadIdx.x;\n'
           + '  const int tid = tid_k_, lane = tid & 63, wave = tid >> 6;\n'
           + f'  const int gtid = blockIdx.x * {BLOCK} + tid;\n'
           + f'  const int nthr = {low.grid} * {BLOCK};\n'
           + f'  const unsigned nblk = {low.grid}u;  // the launch grid (checked at launch)\n'
           + '  unsigned bk_ = 0u;  // grid barriers passed in this launch\n'
           + '  unsigned pk_ = 0u;  // readiness flags published in this launch\n'
           + ''.join(f'  {d}\n' for d in low.decls)
           + (f'  __shared__ unsigned long long ts_sh[{max(1, len(low.sites))}];\n'
              f'  for (int i_ = tid; i_ < {max(1, len(low.sites))}; i_ += {BLOCK}) ts_sh[i_] = 0ull;\n'
              '  __syncthreads();\n'
              '  unsigned long long tlast_ = vh_clock();\n' if timing is True else '')
           + '\n'.join(pre) + '\n'
           + ''.join(f'  {d}\n' for d in low.shared_decls)
           + ''.join(fb_init)
           + (f'  const unsigned TSB_ = {len(low.sites)}u * nblk;  // barrier trace after the site table\n'
              if timing else '')
           + ''.join(f'  for (int e_ = gtid; e_ < {low.fx_words(r) // 2}; e_ += nthr) stz4(rb_S, {low.g[r]}u + 4u * '
                     f'(unsigned)e_);  // both layer buffers of {r}, cleared once a launch\n'
                     for r in sorted(low.fx_parity))
           + ('  grid_sync(bar, nblk, bk_);\n' if low.fx_parity else '')
           + '  for (int st_ = 0; st_ < nsteps; ++st_) {\n'
           + '    const int tid = vh_opaque(tid_k_), lane = tid & 63, wave = tid >> 6;\n'
           + ('    const unsigned bk0_ = bk_;\n' if timing else '')
           + '\n'.join(head) + '\n'
           + '\n'.join(body) + '\n'
           + ('    if (st_ + 1 < nsteps) grid_sync(bar, nblk, bk_);  // feedback visible to the next step\n'
              if low.wrap_barrier else '')
           + '  }\n'
           + ('  __syncthreads();\n'
              f'  for (int i_ = tid; i_ < {len(low.sites)}; i_ += {BLOCK}) TS[i_ * nblk + blockIdx.x] += ts_sh[i_];\n'
              if timing is True else '')
           + ('  grid_exit(bar, nblk);\n}\n' if low.flags_off is None
              else f'  grid_exit_flags(bar, nblk, bar + {low.flags_off}u);\n}}\n'))
    scratch = {}
    for n in low.axes_of:
        r = low.root(n)
        if r in low.g and r not in low.fx:
            axes = low.axes_of[n]
            scratch[n] = (low.g[r], axes, tuple(low.static[a] for a in axes))
    return Lowered(src, params, scratch, low.goff, (low.lds_floats + low.stage_floats) * 4, low.barriers,
                   low.plan, low.sites, low.counters, BLOCK, low.grid, {n: shp for n, (shp, _) in low.res.items()},
                   kernel_name, 1, dict(low.packs), low.history or 0), low
