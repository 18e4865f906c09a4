"""Local folds: a contraction whose fold runs over the points its block has
just made, folded in the same phase instead of after a grid barrier.

The pattern (rows below the matrix-core minimum, fp16 weights):

    u[r.., f] = (fold sum k: A[r.., k] * W1[.., k, f]) + ..   a stream over points f
    g[r.., f] = EPI(u[r.., f])                              its fused epilogue
    y[r.., d] = BASE + fold sum f: g[r.., f] * W2[.., f, d]  BASE additive

The stream gives block b the points f of [b * PPB, (b + 1) * PPB). The
reference lowers y as its own phase, after a grid barrier that makes all of g
visible (``vesta/lower.py:563-600``: a barrier wherever a read sees another
site's writes). Here block b keeps its g values in LDS and folds y over its own
points only: a partial sum for every (row, d) from the rows f of W2 it owns
(W2 in its own layout, d contiguous along a row). Every block adds its
partials, and BASE once per element, into y kept as a 64-bit fixed-point sum
(exact, so the order of the adds changes no bit) in FX_COPIES copies: block b
adds into copy b % FX_COPIES. The rate of atomic adds is limited by the adds
that meet at one address, not by the lines touched, so the copies cut the
time of the adds; a reader sums the copies (exactly). The copies are cleared
in the phase before, right before the barrier that opens the local fold's
phase, so the clear comes after the last read of y's previous value and
before the first add.

One grid barrier per occurrence goes away (GPT-2: the feed-forward
down-projection joins the widening's phase, one barrier per layer fewer).
A lowering that cannot keep a local fold it found (its phase would need a
barrier after all) raises ChainError, and the kernel is lowered again
without local folds.
"""
from __future__ import annotations

from .analysis import LowerError, top_folds
from .mfma import MFMA_ROWS_MIN

FX_COPIES = 4                # copies of a local fold's fixed-point sum (same box, GPT-2 small B=1: 207 / 197 /
                             # 200 / 205 us per step with 2 / 4 / 8 / 16; B=3 274.6 -> 268.7 from 8 to 4;
                             # B=2 239.0 / 241.2, within the spread; with the rotated adds below, four models
                             # each built alternately: 2 / 4 / 8 copies 202.8 / 194.1 / 196.4)
CHAIN_VEC = 8                # weights per 16-byte load (fp16)
CHAIN_STAGE_MAX = 8192       # floats of the block's own values a local fold may keep in LDS
FOLD_ROTATE = 64             # the blocks that add into one copy start their adds this many elements apart
                             # (0: all in the same order; same box, GPT-2 small B=1 with 0 / 64, six models
                             # built alternately, twice: 196.1 / 193.0 us per step; 256 as 64; medium B=1 even)


class ChainError(LowerError):
    """A local fold found by the analysis cannot be kept by the code generation."""


class ChainMixin:
    # ------------------------------------------------------------ analysis
    def find_chains(self, ss):
        """Record every local fold (``chains``: id(y) -> geometry; ``chain_src``:
        id(u) -> the same), keep y as a fixed-point sum in copies and g in the
        producing block's LDS only."""
        for i, s in enumerate(ss):
            if s[0] == 'step':
                self.find_chains(s[6])
                continue
            ch = self.chain_at(ss, i)
            if ch is None:
                continue
            self.chains[id(ch['y'])] = ch
            self.chain_src[id(s)] = ch
            self.chain_local.add(ch['g'])
            self.elided_vals.add(ch['g'])
            self.fx.add(ch['z'])
            self.fx_copies[ch['z']] = FX_COPIES
        # a transposed copy made for y's stream is not read any more
        for ch in self.chains.values():
            W2 = ch['c'].W
            pack = f'{W2}__t'
            others = [k for k, ci in self.info.items()
                      if k != id(ch['y']) and getattr(ci, 'W', None) == W2]
            if pack in self.packs and not others:
                del self.packs[pack]
                self.res.pop(pack, None)

    def chain_at(self, ss, i):
        """The local fold starting at stream ss[i], or None."""
        if i + 2 >= len(ss):
            return None
        s, t, y = ss[i], ss[i + 1], ss[i + 2]
        if s[0] != 'let' or t[0] != 'let' or y[0] != 'let':
            return None
        if self.place.get(id(s)) not in ('tile', 'lane') or self.place.get(id(y)) not in ('tile', 'lane'):
            return None
        if any(id(x) in self.splits or id(x) in self.groups or id(x) in self.elided for x in (s, t, y)):
            return None
        c, c2 = self.info.get(id(s)), self.info.get(id(y))
        if getattr(c, 'kind', None) not in ('tile', 'lane') or getattr(c2, 'kind', None) != 'tile':
            return None
        st = self.stream_of(c)
        if st is None or self.mfma_ok(c, st) or len(st.pts) != 1:
            return None
        reg = list(c.reg_axes)
        R = self.size(reg)
        if R >= MFMA_ROWS_MIN or R > self.REG_MAX:
            return None
        # g: elementwise on u at its own points, read by y alone
        g = t[1]
        if list(t[2]) != list(s[2]) or list(s[2]) != reg + list(st.pts) or top_folds(t[3]):
            return None
        if g in self.outputs or self.root(g) != g or g in self.private or s[1] in self.outputs:
            return None
        if self.readers_of.get(g, set()) != {id(y)}:
            return None
        # y: BASE + fold over u's points of g * W2[.., f, d]
        f = st.pts[0]
        if list(c2.reg_axes) != reg or c2.pt_axes or list(c2.fold_axes) != [f]:
            return None
        if c2.A[0] != 'idx' or c2.A[1] != g or list(c2.A[2]) != [('name', a) for a in t[2]]:
            return None
        shape, dt = self.res[c2.W]
        if dt != 'f16' or c2.widx[-2] != ('name', f):
            return None
        if any(self.free_axes(x) & ({f, c2.contig} | set(reg)) for x in c2.widx[:-2]):
            return None
        d = c2.contig
        if d in self.dynamic or f in self.dynamic:
            return None
        D = self.static[d]
        if D % CHAIN_VEC or shape[-1] % CHAIN_VEC or D // CHAIN_VEC > (self.NWAVE - 1) * 64:
            return None
        if not self._additive(c2.epi, ('name', '__acc'), '__acc'):
            return None
        z = self.root(y[1])
        if y[1] in self.outputs or z in self.outputs or z in self.private or z in self.fx:
            return None
        if list(y[2]) != reg + [d] or list(self.axes_of[z]) != list(y[2]):
            return None
        P = self.size(st.pts)
        PPB = -(-P // self.grid)
        if R * PPB > CHAIN_STAGE_MAX:
            return None
        base = self.rebuild_expr(c2.epi, lambda n: ('num', 0.0) if n == ('name', '__acc') else n)
        return dict(u=s, gs=t, y=y, c=c2, g=g, z=z, f=f, d=d, P=P, PPB=PPB, R=R, D=D, reg=reg, base=base)

    # ------------------------------------------------------------ readiness flags
    def ready_point(self, what, ranges, active, out, ind, made, setup=()):
        """Instead of a grid barrier before ``what``: every block publishes
        that what it stored so far is complete, then waits only for the blocks
        it reads from: ``ranges`` is a list of (first, last) C expressions of
        producer blocks (clamped to the grid), ``active`` a C condition (a
        block that is not active waits for none). Between the two, a prefetch
        slot takes the loads issued early for the next sites, as between a
        grid barrier's arrival and wait."""
        if self.flags_off is None:
            self.flags_off = self.alloc_counters(self.grid)
        F = self.flags_off
        out.append(f'{ind}pk_ += 1u; flag_publish(bar + {F}u, pk_);  // {made} stored: {what} waits for its makers')
        self.mark(out, ind, f'publish before {what}')
        self.pf_open(out, ind, self.dirty, self.readers)
        self.pf_slots[-1]['ready'] = True
        if len(ranges) > 4:
            raise ChainError(f'{what}: more than four producer ranges')
        I = ind + '  '
        out.append(f'{ind}{{')
        out += [I + x for x in setup]
        args = []
        for q, (lo, hi) in enumerate(ranges):
            out.append(f'{I}const int a{q}_ = {lo}, n{q}_ = ({active}) ? min({hi}, (int)nblk - 1) - a{q}_ + 1 : 0;')
            args += [f'a{q}_', f'n{q}_']
        out.append(f'{I}flag_wait(bar, bar + {F}u, pk_, {", ".join(args)}); }}')
        self.mark(out, ind, f'wait before {what}')

    # ------------------------------------------------------------ storage
    def fx_copy_stride(self, z):
        """Floats between copies of fixed-point sum z (16-byte aligned)."""
        return -(-2 * max(1, self.size(self.axes_of[z])) // 4) * 4

    def fx_words(self, z):
        """Floats of global scratch fixed-point sum z takes (all its copies)."""
        return self.fx_copy_stride(z) * self.fx_copies.get(z, 1)

    def gofs(self, r, ahead=0):
        """C expression: the float offset of fixed-point sum r in global
        scratch. A sum kept in two buffers by layer parity (``fx_parity``;
        layers counted across the steps of a launch, st_ * n + l) has the
        buffer of the current layer (``ahead`` 1: of the next one); after its
        layer loop, the buffer the loop's last layer left."""
        if r not in self.fx_parity:
            return f'{self.g[r]}u'
        lv, var, n, _ = self.fx_parity[r]
        layer = lv if any(lp['var'] == var for lp in self.loops) else str(n)
        return f'({self.g[r]}u + (unsigned)((st_ * {n} + {layer} + {ahead}) & 1) * {self.fx_words(r)}u)'

    def gadd(self, r):
        """C expression: the offset the current layer's atomic adds into r go
        to: the current buffer, or for a layer loop's carry (read as the
        previous layer left it, added into for the next layer) the next one."""
        carry = r in self.fx_parity and self.fx_parity[r][3] == 'carry'
        return self.gofs(r, ahead=1 if carry else 0)

    def fx_copy_base(self, z):
        """C expression: float offset of the copy the current block adds into."""
        C = self.fx_copies.get(z, 1)
        return f'(unsigned)(blockIdx.x % {C}u) * {self.fx_copy_stride(z)}u' if C > 1 else '0u'

    # ------------------------------------------------------------ code generation
    def chain_clear(self, z, out, ind):
        """Clear z's copies right before the barrier that opened this phase.
        That barrier must not be the first of its loop body, and neither the
        phase it closes nor this one may touch z before here. A layer loop's
        carry in parity buffers is cleared here instead: the buffer this
        layer's reads took (in an earlier phase), which the next layer's adds
        will use."""
        if z in self.fx_parity and self.fx_parity[z][3] == 'carry':
            self.trace.append(('clear', z, None, 0))
            n4 = self.fx_words(z) // 4
            out.append(f'{ind}for (int e_ = (int)blockIdx.x + (int)nblk * tid; e_ < {n4}; e_ += nthr) '
                       f'stz4(rb_S, {self.gofs(z)} + 4u * (unsigned)e_);  // clear the buffer of {z} read '
                       f'before, for the next layer')
            return
        k, loop = self.last_pf, self.loop_id()
        if k is None or self.pf_slots[k].get('ready'):
            raise ChainError(f'local fold into {z}: no grid barrier right before its phase')
        slot = self.pf_slots[k]
        if slot['loop'] != loop or not any(self.pf_slots[j]['loop'] == loop for j in range(k)):
            raise ChainError(f'local fold into {z}: its phase is the first of a loop body')
        if z in slot['readers'] or z in slot['dirty'] or z in self.readers or z in self.dirty:
            raise ChainError(f'local fold into {z}: {z} is used in the phase before')
        n4 = self.fx_words(z) // 4
        self.trace.append(('clear', z, k, 0))
        slot['pre'].append(f'for (int e_ = (int)blockIdx.x + (int)nblk * tid; e_ < {n4}; e_ += nthr) '
                           f'stz4(rb_S, {self.g[z]}u + 4u * (unsigned)e_);  // clear the copies of {z}')

    def chain_base(self, ch, out, ind):
        """BASE into y's fixed-point sum, once per element over all blocks (an
        atomic add: other blocks' partials may already be in)."""
        z = ch['z']
        axes = list(ch['axes']) if 'axes' in ch else ch['reg'] + [ch['d']]
        if 'sz' in ch:
            self.plan.append((self.show_stmt(ch['sz']), 'fixed-point sum in two layer buffers: base and '
                              'projection added'))
        early = self.early_spread_loads(axes, ch['base'], out, ind)
        self.trace.append(('adds', z, frozenset(self.root_reads([ch['base']]))))
        I = ind + '  '
        out.append(f'{ind}{{ const unsigned cz_ = {self.fx_copy_base(z)};')
        out.append(f'{ind}for (int p_ = (int)blockIdx.x + (int)nblk * tid; p_ < {self.count_c(axes)}; '
                   f'p_ += nthr) {{  // {z} base')
        env = self.decode('p_', axes, out, I)
        pre = []
        v, t = self.spread_value(ch['base'], env, pre, I, early)
        out += pre
        out.append(f'{I}fxadd(S, {self.gadd(z)} + cz_ + 2u * (unsigned)p_, {self.as_float(v, t)});')
        out.append(f'{ind}}} }}')
        ch['base_done'] = True
        self.mark(out, ind, f'{z} base')

    def gen_chain(self, y, ch, out, ind):
        c, z, g = ch['c'], ch['z'], ch['g']
        R, D, P, PPB, reg = ch['R'], ch['D'], ch['P'], ch['PPB'], ch['reg']
        held = self.chain_lds.pop(g, None)
        if held is None or held[1] != PPB or held[2] != R:
            raise ChainError(f'local fold {y[1]}: {g} is not in the LDS of the blocks that made it')
        gbase = held[0]
        reads = self.root_reads([ch['base']])
        nb = self.barriers
        self.sync(reads, {z}, out, ind, y[1])
        if self.barriers != nb:
            raise ChainError(f'local fold {y[1]}: its phase would need a barrier after {ch["u"][1]}')
        self.chain_clear(z, out, ind)
        self.plan.append((self.show_stmt(y), f'local fold over the points of {ch["u"][1]} '
                          f'({PPB} per block), fixed-point sum in {self.fx_copies[z]} copies'))
        NW = self.NWAVE - 1
        VEC = CHAIN_VEC
        NCH = D // VEC                        # 16-byte column chunks of a W2 row
        RG = max(1, min(PPB, (NW * 64) // NCH))   # row groups: thread tid folds chunk tid % NCH of
        RPG = -(-PPB // RG)                   # rows tid / NCH, + RG, .. of the block's own
        NT = NCH * RG
        W = c.W
        rr, rs = self.rsrc(W), self.res_strides(W)
        kept = self.weights_kept('stream')
        prefetch = RPG * 4 <= self.pf_budget
        sid = self.fresh('c')
        wc = f'wc_{sid}'
        role = [f'const int cc_ = tid % {NCH}, cg_ = tid / {NCH};',
                f'const int f0_ = (int)blockIdx.x * {PPB}, nf_ = min({PPB}, {P} - f0_);']

        def wload(i, dst, step_override):
            saved = self.override_step(step_override)
            try:
                lines = [f'{{ const int fl_ = cg_ + {i * RG};',
                         f'  if (tid < {NT} && fl_ < nf_) {{']
                env = {ch['f']: ('(f0_ + fl_)', 'int'), ch['d']: (f'(cc_ * {VEC})', 'int')}
                pre = []
                ix = [self.index(x, env, pre, '    ') for x in c.widx]
                lines += pre
                a = self.addr(ix, rs)
                lines.append(f'    {dst} = {self.nt_load("f16", VEC, rr, f"(unsigned)({a})", kept)};')
                lines.append(f'  }} else {dst} = vh_u32x4{{0u, 0u, 0u, 0u}};')
                lines.append('}')
                return lines
            finally:
                self.restore_step(saved)

        if prefetch:
            self.decls.append(f'vh_u32x4 {wc}[{RPG}];')

            def make(step_override):
                lines = [f'if (wave < {NW}) {{'] + ['  ' + x for x in role]
                for i in range(RPG):
                    lines += ['  ' + x for x in wload(i, f'{wc}[{i}]', step_override)]
                return lines + ['}']
            self.place_prefetch(make, out, ind)
        I = ind + '  '
        o = out
        o.append(f'{ind}{{  // local fold {y[1]}: {PPB} points of {ch["u"][1]} per block x {D} from {W}, '
                 f'rows={R}, {RG} row groups of {RPG}' + (' prefetched' if prefetch else ''))
        o += [I + x for x in role]
        if not prefetch:
            o.append(f'{I}vh_u32x4 {wc}[{RPG}];')
            for i in range(RPG):
                o += [I + x for x in wload(i, f'{wc}[{i}]', None)]
        red = -(-(gbase + R * PPB) // 4) * 4
        self.stage_floats = max(self.stage_floats, red + RG * R * D - self.lds_floats)
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}float ac_[{R}][{VEC}];')
        o.append(f'{I}#pragma unroll')
        o.append(f'{I}for (int r_ = 0; r_ < {R}; ++r_)')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int v_ = 0; v_ < {VEC}; ++v_) ac_[r_][v_] = 0.0f;')
        o.append(f'{I}if (tid < {NT}) {{')
        for i in range(RPG):
            o.append(f'{I}  {{ const int fl_ = cg_ + {i * RG};')
            o.append(f'{I}    if (fl_ < nf_) {{')
            o.append(f'{I}      float wf_[{VEC}];')
            o.append(f'{I}      unpack8({wc}[{i}], wf_);')
            o.append(f'{I}      #pragma unroll')
            o.append(f'{I}      for (int r_ = 0; r_ < {R}; ++r_) {{')
            o.append(f'{I}        const float gv_ = sh_f[{gbase} + r_ * {PPB} + fl_];')
            o.append(f'{I}        #pragma unroll')
            o.append(f'{I}        for (int v_ = 0; v_ < {VEC}; ++v_) ac_[r_][v_] = fmaf(gv_, wf_[v_], ac_[r_][v_]);')
            o.append(f'{I}      }}')
            o.append(f'{I}    }}')
            o.append(f'{I}  }}')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int r_ = 0; r_ < {R}; ++r_) {{')
        o.append(f'{I}    float* dq_ = sh_f + {red} + (cg_ * {R} + r_) * {D} + cc_ * {VEC};')
        o.append(f'{I}    *(vh_f32x4*)dq_ = vh_f32x4{{ac_[r_][0], ac_[r_][1], ac_[r_][2], ac_[r_][3]}};')
        o.append(f'{I}    *(vh_f32x4*)(dq_ + 4) = vh_f32x4{{ac_[r_][4], ac_[r_][5], ac_[r_][6], ac_[r_][7]}};')
        o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        self.mark(o, I, f'local fold {y[1]}: partials')
        # the row groups' partials, added in group order, into the block's copy
        o.append(f'{I}if (nf_ > 0) {{')
        o.append(f'{I}  const unsigned cz_ = {self.fx_copy_base(z)};')
        if FOLD_ROTATE:
            # the blocks sharing a copy start at different elements, so that
            # their adds do not queue at the same lines at once (any order of
            # integer adds gives the same sum)
            C = self.fx_copies.get(z, 1)
            o.append(f'{I}  const int ro_ = (int)((blockIdx.x / {C}u) * {FOLD_ROTATE}u % {R * D}u);')
            o.append(f'{I}  for (int i_ = tid; i_ < {R * D}; i_ += {self.BLOCK}) {{')
            o.append(f'{I}    const int e_ = i_ + ro_ < {R * D} ? i_ + ro_ : i_ + ro_ - {R * D};')
        else:
            o.append(f'{I}  for (int e_ = tid; e_ < {R * D}; e_ += {self.BLOCK}) {{')
        o.append(f'{I}    float v_ = sh_f[{red} + e_];')
        for q in range(1, RG):
            o.append(f'{I}    v_ += sh_f[{red} + {q * R * D} + e_];')
        o.append(f'{I}    fxadd(S, {self.gadd(z)} + cz_ + 2u * (unsigned)e_, v_);')
        o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')
        if not ch.get('base_done'):
            self.chain_base(ch, out, ind)
        self.note(reads, {z})
        self.mark(out, ind, f'local fold {y[1]}')
