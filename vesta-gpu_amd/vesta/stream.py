"""Streamed contractions: one weight row per output point, read along the fold.

A sum contraction ``y[.., p] = fold sum k: A[r, k] * W[.., k-or-p ..]`` whose
weight is a read-only residue is lowered so that every output point reads
one contiguous row of K weights:

  * ``lane`` pattern (the fold indexes W's last axis, e.g. the LM head
    ``wte[n, d]``): rows are W's own rows;
  * ``tile`` pattern (the output axis indexes W's last axis, e.g.
    ``qkvw[l, d, j]``): the kernel reads a copy of W transposed in its last
    two axes (``<W>__t``), made once when the residues are bound, so column
    ``j`` of W becomes a contiguous row.

Points are split into equal contiguous ranges, one per block (no split-K, so
no partial sums cross blocks); inside a block each wave takes ``64 / lpp``
points at a time, ``lpp`` lanes per point, 16-byte loads along the fold and a
butterfly reduction. The other factor is read from LDS (in place when it is a
block-private value laid out [rows, fold], otherwise staged there first).

When a block's share of the weights fits in a few registers, its loads are
issued ahead of time: at the grid barrier before the site, between
``grid_arrive`` and ``grid_wait`` (or, for the first site of a layer loop,
at the end of the previous iteration), so the weights are in flight while
the block waits for the values they multiply.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

PREFETCH_VGPRS = 64          # registers per lane one site may hold prefetched weights in (default budget)
PROJ_KEPT_BYTES = 64 << 20   # out-projection weights (all layers) kept in the caches up to this size
PI_STREAM = 2                # slots whose loads are issued together when not prefetched
PB_MAX = 2                   # points one lane group makes at once (each LDS read of the other factor serves them all)
                             # (B=1, the output head's stream: 229 us per step at 4 and 4, 219 at 2 and 2)
PB_ACC = 32                  # ... holding at most this many partial sums per lane
STREAM_ALL_WAVES = True      # a stream whose weights are not prefetched runs on every wave, the polling one
                             # too (it polls nothing while the stream runs)
STAGE_OUT_MAX = 8192         # floats of a stream's values a block collects in LDS before writing them out


@dataclass
class Stream:
    pack: str | None          # name of the transposed copy, or None (rows are W's own)
    src: str                  # the residue read (W or its copy)
    K: int                    # fold length (flattened fold axes)
    c0: int                   # first fold element within a row
    rowlen: int               # row length of the array read
    prefix_idx: list          # index expressions of the leading axes, the point's own axis last (tile)
    pts: list                 # point axes (row-major)
    vec: int                  # elements per load


class StreamMixin:
    # ------------------------------------------------------------ eligibility
    def stream_of(self, c):
        """Stream description of contraction c, or None when it cannot stream."""
        W = c.W
        shape, dt = self.res[W]
        if W in self.emitted or W in self.fb_targets or dt not in ('f16', 'f32'):
            return None
        if any(a in self.dynamic for a in c.fold_axes) or any(a in self.dynamic for a in c.pt_axes):
            return None
        K = math.prod(self.static[a] for a in c.fold_axes)
        if c.kind == 'lane':
            if len(c.fold_axes) != 1 or c.widx[-1] != ('name', c.fold_axes[0]):
                return None
            rowlen, c0, pack = shape[-1], 0, None
            prefix = list(c.widx[:-1])
            pts = list(c.pt_axes)
        else:
            if len(shape) < 2 or c.contig in self.dynamic:
                return None
            aff = self.affine(c.widx[-2])
            if aff is None:
                return None
            const, coefs = aff
            stride = 1
            for a in reversed(c.fold_axes):
                if coefs.get(a) != stride:
                    return None
                stride *= self.static[a]
            if set(coefs) != set(c.fold_axes) or const < 0 or const + K > shape[-2]:
                return None
            for x in c.widx[:-2]:
                if self.free_axes(x) & (set(c.fold_axes) | {c.contig}):
                    return None
            rowlen, c0 = shape[-2], const
            pack = f'{W}__t'
            prefix = list(c.widx[:-2]) + [('name', c.contig)]
            pts = list(c.pt_axes) + [c.contig]
        esz = 2 if dt == 'f16' else 4
        vec = next(v for v in ((8, 4, 2, 1) if esz == 2 else (4, 2, 1))
                   if K % v == 0 and rowlen % v == 0 and c0 % v == 0)
        if pack is not None and pack not in self.res:
            self.res[pack] = (tuple(shape[:-2]) + (shape[-1], shape[-2]), dt)
            self.packs[pack] = W
        return Stream(pack, pack or W, K, c0, rowlen, prefix, pts, vec)

    # ------------------------------------------------------------ prefetch slots
    def pf_open(self, out, ind, dirty=(), readers=()):
        """A place for prefetch code between grid_arrive and grid_wait (and
        one before grid_arrive, ``pre``, for code that must end before the
        block arrives). ``dirty`` / ``readers``: values written / read since
        the previous barrier (other blocks' writes of them are not yet
        visible there)."""
        k = len(self.pf_slots)
        self.pf_slots.append({'lines': [], 'pre': [], 'loop': self.loop_id(), 'ind': ind, 'dirty': set(dirty),
                              'readers': set(readers)})
        out.append(f'/*@PF{k}@*/')
        self.last_pf = k

    def loop_id(self):
        return self.loops[-1]['id'] if self.loops else None

    def prefetch_target(self):
        """Where code issued early for the next site goes: ('slot', k) for the
        latest barrier of this loop body, ('loop', k) for the barrier before
        the loop (plus the end of the previous iteration), ('top', None) when
        the loop has no barrier before it (in place in the first iteration,
        plus the end of the previous one), or None (in place)."""
        k = self.last_pf
        if k is not None and self.pf_slots[k]['loop'] == self.loop_id():
            return 'slot', k
        lp = self.loops[-1] if self.loops else None
        if lp is not None and k == lp['pf_before'] and not lp['body_barrier']:
            return ('loop', k) if k is not None else ('top', None)
        return None

    def unsafe_early(self):
        """Values that early loads must not read: written after the barrier
        before the one the loads go to."""
        tgt = self.prefetch_target()
        bad = set(self.dirty)
        if tgt is not None:
            if tgt[1] is not None:
                bad |= self.pf_slots[tgt[1]]['dirty']
            if tgt[0] in ('loop', 'top'):
                bad |= self.loops[-1]['end_dirty']
        return bad

    def place_prefetch(self, make, out, ind):
        """Put the prefetch code ``make(step_override)`` (a list of lines) at the
        latest barrier of this loop body, or before the loop and at the end of
        the previous iteration; with no barrier to use, in place."""
        tgt = self.prefetch_target()
        if tgt is None:
            out += [ind + x for x in make(None)]
            return
        kind, k = tgt
        if kind == 'slot':
            self.pf_slots[k]['lines'] += make(None)
            return
        lp = self.loops[-1]
        lv, n = lp['lv'], lp['n']
        if kind == 'loop':
            self.pf_slots[k]['lines'] += make(('0', 'int'))
        else:
            out.append(f'{ind}if ({lv} == 0) {{')
            out += [ind + '  ' + x for x in make(('0', 'int'))]
            out.append(f'{ind}}}')
        nxt = make((f'({lv} + 1)', 'int'))
        lp['end_prefetch'] += [f'if ({lv} + 1 < {n}) {{'] + ['  ' + x for x in nxt] + ['}']

    # ------------------------------------------------------------ codegen
    def gen_stream(self, s, c, st, fused, out, ind):
        if self.mfma_ok(c, st) and self.mfma_reachable(c, st):
            return self.gen_stream_mfma(s, c, st, fused, out, ind)
        name = s[1]
        ch = self.chain_src.get(id(s))
        if ch is not None and [(k, id(t)) for k, t, _ in fused] != [('let', id(ch['gs']))]:
            from .chain import ChainError
            raise ChainError(f'local fold {ch["y"][1]}: {ch["g"]} is not the epilogue of {name}')
        reads, writes = self.site_io(s, c, fused)
        if ch is not None:
            writes.discard(ch['g'])           # kept in the block's LDS only
        self.sync(reads, writes, out, ind, name)
        self.plan.append((self.show_stmt(s), 'stream' + (' (transposed copy)' if st.pack else '')
                          + (f' +{len(fused)} fused' if fused else '')))
        for _, t, _ in fused:
            self.plan.append((self.show_stmt(t), f'epilogue of {name}'))
        dt = self.res[st.src][1]
        esz = 2 if dt == 'f16' else 4
        vec, K = st.vec, st.K
        nv = K // vec
        lpp = 64
        while lpp > 1 and (nv % lpp != 0 or nv < lpp):
            lpp //= 2
        if lpp < 8 and nv >= 64:
            lpp = 64
        pl = -(-nv // lpp)
        exact = nv % lpp == 0
        ppw = 64 // lpp
        NW = self.NWAVE - 1          # compute waves; the last wave polls barriers and holds no early loads
        P = self.size(st.pts)
        NB = self.grid
        PPB = -(-P // NB)
        reg = c.reg_axes
        R = self.size(reg)
        rch = min(R, self.REG_MAX)
        nrch = -(-R // rch)
        ltype = self.load_type(dt, vec)
        vregs = -(-PPB // (NW * ppw)) * pl * max(1, vec * esz // 4)
        prefetch = vregs <= self.pf_budget
        if not prefetch and STREAM_ALL_WAVES and ch is None:
            NW = self.NWAVE
        # a long stream with several rows: a lane group makes PB points at once,
        # so each value of the other factor read from LDS serves PB weight
        # vectors (a short one keeps every wave busy instead)
        PB = 1 if rch < 4 or prefetch else max(1, min(PB_MAX, PPB, PB_ACC // rch))
        NQ = -(-PPB // (NW * ppw * PB))
        sid = self.fresh('s')
        wq = f'wq_{sid}'
        I = ind + '  '
        o = out

        geo = dict(P=P, PPB=PPB, NW=NW, ppw=ppw, lpp=lpp, rch=rch, reg=reg, PB=PB)

        def load_lines(q_c, dst, step_override):
            """Lines loading slot q_c's vectors into dst[j][m] (j < PB, m < pl)."""
            lines = []
            saved = None
            if step_override is not None:
                saved = dict(self.step_env)
                for v in list(self.step_env):
                    if self.loops and v == self.loops[-1]['var']:
                        self.step_env[v] = step_override
            for j in range(PB):
                p_c, ok_c = self.slot_point(geo, q_c, j)
                lines.append(f'{{ const int p_ = {p_c};')
                lines.append(f'  if ({ok_c} && p_ < {P}) {{')
                env = self.decode('p_', st.pts, lines, '    ', prefix='sp_')
                pre = []
                ix = [self.index(x, env, pre, '    ') for x in st.prefix_idx]
                lines += pre
                rs = self.res_strides(st.src)
                base = self.addr(ix, rs[:-1]) if ix else '0'
                lines.append(f'    const unsigned wr_ = (unsigned)({base}) + {st.c0}u;')
                lines.append('    #pragma unroll')
                lines.append(f'    for (int m_ = 0; m_ < {pl}; ++m_) {{')
                lines.append(f'      const int kv_ = cl_ + m_ * {lpp};')
                cond = '' if exact else f'if (kv_ < {nv}) '
                lines.append(f'      {cond}{dst}[{j}][m_] = '
                             f'{self.nt_load(dt, vec, self.rsrc(st.src), "wr_ + kv_ * %d" % vec, self.weights_kept("stream"))};')
                if not exact:
                    lines.append(f'      else {dst}[{j}][m_] = {self.vec_zero(dt, vec)};')
                lines.append('    }')
                lines.append('  } else {')
                lines.append('    #pragma unroll')
                lines.append(f'    for (int m_ = 0; m_ < {pl}; ++m_) {dst}[{j}][m_] = {self.vec_zero(dt, vec)};')
                lines.append('  }')
                lines.append('}')
            if saved is not None:
                self.step_env.clear()
                self.step_env.update(saved)
            return lines

        lane_decl = [f'const int sub_ = lane / {lpp}, cl_ = lane % {lpp};']
        rows_of = [min(rch, R - rc * rch) for rc in range(nrch)]
        self.geo_nw = NW
        if prefetch:
            self.decls.append(f'{ltype} {wq}[{NQ}][{PB}][{pl}];')
            unsafe = self.unsafe_early()
            caps = {}

            def make(step_override):
                """Weights of every slot, and the loads of the epilogues that may
                be issued early, into registers."""
                lines = [f'if (wave < {NW}) {{'] + ['  ' + x for x in lane_decl]
                for q in range(NQ):
                    lines += ['  ' + x for x in load_lines(str(q), f'{wq}[{q}]', step_override)]
                saved = self.override_step(step_override)
                for rc in range(nrch):
                    for q in range(NQ):
                        for j in range(-(-(rows_of[rc] * PB) // lpp)):
                            pre = f'pf_{sid}_{q}_{rc}_{j}_'
                            loads = self.epi_loads(s, c, st, fused, geo, str(q), rc, j, rows_of[rc], pre, unsafe)
                            caps[pre] = [(n, k) for n, _, k in loads]
                            if loads:
                                lines += ['  ' + x for x in self.epi_context(st, geo, str(q), rc, j, rows_of[rc],
                                                                               [f'{n} = {t};' for n, t, _ in loads])]
                self.restore_step(saved)
                return lines + ['}']
            self.place_prefetch(make, o, ind)
            for pre, regs in caps.items():
                for n, k in regs:
                    self.decls.append(f'{self.cap_ctype(k)} {n};')
        o.append(f'{ind}{{  // stream {name}: {P} points x {K} from {st.src}, VEC={vec} lanes/point={lpp} '
                 f'points/block={PPB} rows={R} points/lane group={PB}{" prefetched" if prefetch else ""}')
        for x in lane_decl:
            o.append(f'{I}{x}')
        # which block made which points (an argmax over them can stay in the block)
        self.stream_part[self.root(name)] = dict(pts=list(st.pts), PPB=PPB, P=P, reg=list(reg))
        # the other factor, as floats in LDS laid out [row, fold]
        direct = self.direct_lds(c, reg)
        # values of the site: not stored when only its own epilogue reads them;
        # with several rows (or an argmax reading them next), collected in LDS
        # [row][own point] and written out row by row afterwards
        fused_ids = {id(t) for _, t, _ in fused}
        made = [s] + [t for kind, t, _ in fused if kind == 'let']
        self.skip_store = {t[1] for t in made if self.epi_only(t[1], fused_ids)}
        self.out_stage = {}
        obase = self.lds_floats + self.stage_top + (0 if direct is not None else rch * K)
        otop = obase
        for t in made:
            n = t[1]
            if n in self.skip_store or not self.stage_out_ok(t, reg, st.pts, R, PPB):
                continue
            self.out_stage[n] = (otop, PPB, list(reg), list(st.pts))
            otop += -(-R * PPB // 4) * 4
        self.stage_floats = max(self.stage_floats, otop - self.lds_floats)
        for rc in range(nrch):
            if direct is not None:
                abase = f'{direct} + {rc * rch * K}'
            else:
                abase = str(self.lds_floats + self.stage_top)
                self.stage_floats = max(self.stage_floats, self.stage_top + rch * K)
                self.stage_A(c, reg, rc, rch, R, K, abase, o, I)
                self.mark(o, I, f'stream {name}: stage')
            qs = [str(q) for q in range(NQ)] if prefetch else None
            self.stream_body(s, c, st, fused, o, I, rc, rch, R, K, abase, dt, vec, nv, lpp, pl, exact,
                             NQ, qs, wq, ltype, geo, load_lines, sid, unsafe if prefetch else None)
        if any(n not in self.chain_local for n in self.out_stage):
            self.write_out(P, PPB, R, o, I)
            self.mark(o, I, f'stream {name}: write out')
        self.stream_lds = {self.root(n): (base, PPB, R) for n, (base, _, _, _) in self.out_stage.items()}
        self.chain_lds = {n: (base, PPB, R) for n, (base, _, _, _) in self.out_stage.items()
                          if n in self.chain_local}
        self.skip_store, self.out_stage = set(), {}
        o.append(f'{ind}}}')
        self.note(reads, writes)
        self.mark(out, ind, f'stream {name}')

    def write_out(self, P, PPB, R, o, I):
        """The block's LDS copies of its values ([row][own point]) into global
        scratch, row by row (consecutive threads, consecutive points)."""
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}{{ const int p0_ = (int)blockIdx.x * {PPB};')
        o.append(f'{I}  for (int e_ = tid; e_ < {R * PPB}; e_ += {self.BLOCK}) {{')
        o.append(f'{I}    const int r_ = e_ / {PPB}, i_ = e_ - r_ * {PPB};')
        o.append(f'{I}    if (p0_ + i_ < {P}) {{')
        for n, (base, _, _, _) in self.out_stage.items():
            if n in self.chain_local:
                continue
            o.append(f'{I}      stcs(rb_S, {self.g[self.root(n)]} + r_ * {P} + p0_ + i_, sh_f[{base} + e_]);')
        o.append(f'{I}    }}')
        o.append(f'{I}  }}')
        o.append(f'{I}}}')

    def epi_only(self, n, fused_ids):
        """Is value n read only by the statements fused into this epilogue?"""
        r = self.root(n)
        carries = set(self.alias) | set(self.alias.values())
        return (n not in self.outputs and r == n and n not in carries
                and self.readers_of.get(n, set()) <= fused_ids)

    def stage_out_ok(self, t, reg, pts, R, PPB):
        """Can value t (made at every point of this stream) go through an LDS
        copy: laid out [reg axes, point axes] in global scratch, and worth it
        (several rows per point, or the argmax that reads it next)?"""
        n = t[1]
        r = self.root(n)
        if n in self.chain_local:
            return list(t[2]) == list(reg) + list(pts)
        if r in self.private or r in self.fx or r not in self.g or list(self.axes_of[r]) != list(t[2]):
            return False
        if list(t[2]) != list(reg) + list(pts) or R * PPB > STAGE_OUT_MAX:
            return False
        return R >= 2 or any(i in self.argmax for i in self.readers_of.get(n, ()))

    def override_step(self, step_override):
        saved = dict(self.step_env)
        if step_override is not None and self.loops:
            self.step_env[self.loops[-1]['var']] = step_override
        return saved

    def restore_step(self, saved):
        self.step_env.clear()
        self.step_env.update(saved)

    @staticmethod
    def slot_point(geo, q, j='0'):
        """(point, valid) of point j of this lane group in slot q: a lane group
        makes PB consecutive points of its block's range."""
        NW, ppw, PPB, PB = geo['NW'], geo['ppw'], geo['PPB'], geo['PB']
        loc = f'(({q} * {NW} + wave) * {ppw} + sub_) * {PB} + {j}' if PB > 1 else \
            f'({q} * {NW} + wave) * {ppw} + sub_'
        return f'((int)blockIdx.x * {PPB} + {loc})', f'(wave < {NW} && {loc} < {PPB})'

    def epi_item(self, geo, q_c, t, rows, lines, ind):
        """Lines binding item t of this lane: after the butterfly every lane of
        a group holds all (point, row) sums; item it_ = cl_ + t * lpp of the
        group's PB * rows is point jj_, row r_. Returns (point, valid)."""
        PB = geo['PB']
        lines.append(f'{ind}const int it_ = cl_ + {t * geo["lpp"]};')
        if PB > 1:
            lines.append(f'{ind}const int jj_ = it_ / {rows}, r_ = it_ % {rows};')
        else:
            lines.append(f'{ind}const int jj_ = 0, r_ = it_;')
        p_c, ok_c = self.slot_point(geo, q_c, 'jj_')
        return p_c, f'it_ < {rows * PB} && {ok_c}'

    def epi_context(self, st, geo, q_c, rc, j, rows, body):
        """Lines binding the point and row of this lane's item j of slot q_c
        around ``body`` (lines that may use them)."""
        lines = ['{']
        p_c, ok = self.epi_item(geo, q_c, j, rows, lines, '  ')
        lines += [f'  const int p_ = {p_c};', f'  if ({ok} && p_ < {geo["P"]}) {{']
        self.decode('p_', st.pts, lines, '    ', prefix='ep_')
        if geo['reg']:
            self.decode(f'({rc * geo["rch"]} + r_)', geo['reg'], lines, '    ', prefix='er_')
        lines += ['    ' + x for x in body]
        lines += ['  }', '}']
        return lines

    def epi_env(self, st, geo, rc):
        env = {a: (f'ep_{a}', 'int') for a in st.pts}
        for a in geo['reg']:
            env[a] = (f'er_{a}', 'int')
        return env

    def epi_loads(self, s, c, st, fused, geo, q_c, rc, j, rows, prefix, unsafe):
        """The loads the epilogue of (slot, row chunk, lane group member j)
        would issue that may go early: (register, load expression, kind)."""
        self.capture = {'prefix': prefix, 'loads': [], 'unsafe': unsafe}
        try:
            self.epilogue(s, c, fused, self.epi_env(st, geo, rc), '0.0f', [], '')
            return self.capture['loads']
        finally:
            self.capture = None

    def stream_body(self, s, c, st, fused, o, I, rc, rch, R, K, abase, dt, vec, nv, lpp, pl, exact,
                    NQ, qs, wq, ltype, geo, load_lines, sid, unsafe):
        """The dot products of one row chunk, then the epilogues. ``qs``: the
        slots as compile-time constants when the weights were prefetched (the
        epilogue then reads early-issued registers), else None (slots are
        streamed PI_STREAM at a time)."""
        rows = min(rch, R - rc * rch)
        PB = geo['PB']
        rpl = -(-(rows * PB) // lpp)
        J2 = I + '  '
        if qs is None:
            # groups of PI slots, software-pipelined: the loads of the next group
            # are in flight while the current one is multiplied and reduced (two
            # named register buffers, the loop unrolled by two: a copy between
            # buffers would wait for the loads it copies)
            PI = max(1, PI_STREAM // PB)

            def issue(buf, q0):
                lines = []
                for qi in range(PI):
                    lines.append(f'if ({q0} + {qi} < {NQ}) {{')
                    lines += ['  ' + x for x in load_lines(f'({q0} + {qi})', f'{buf}[{qi}]', None)]
                    lines.append('}')
                return lines

            def consume(buf, q0, ind2):
                o.append(f'{ind2}#pragma unroll')
                o.append(f'{ind2}for (int qi_ = 0; qi_ < {PI}; ++qi_) {{')
                K3 = ind2 + '  '
                o.append(f'{K3}const int q_ = {q0} + qi_;')
                o.append(f'{K3}if (q_ >= {NQ}) break;')
                self.slot_dot(o, K3, 'q_', f'{buf}[qi_]', dt, vec, nv, lpp, pl, exact, rch, K, abase, geo)
                self.slot_epilogue(s, c, st, fused, o, K3, 'q_', rc, rows, rpl, geo, None)
                o.append(f'{ind2}}}')
            o.append(f'{I}{{')
            o.append(f'{J2}{ltype} wl_[{PI}][{PB}][{pl}], wn_[{PI}][{PB}][{pl}];')
            o += [J2 + x for x in issue('wl_', '0')]
            o.append(f'{J2}for (int q0_ = 0; q0_ < {NQ}; q0_ += {2 * PI}) {{')
            K2 = J2 + '  '
            o += [K2 + x for x in issue('wn_', f'(q0_ + {PI})')]
            consume('wl_', 'q0_', K2)
            o += [K2 + x for x in issue('wl_', f'(q0_ + {2 * PI})')]
            o.append(f'{K2}if (q0_ + {PI} < {NQ}) {{')
            consume('wn_', f'(q0_ + {PI})', K2 + '  ')
            o.append(f'{K2}}}')
            o.append(f'{J2}}}')
            o.append(f'{I}}}')
            return
        for q in qs:
            o.append(f'{I}{{  // slot {q}')
            self.slot_dot(o, J2, q, f'{wq}[{q}]', dt, vec, nv, lpp, pl, exact, rch, K, abase, geo)
            self.mark(o, J2, f'stream {s[1]}: dot')
            self.slot_epilogue(s, c, st, fused, o, J2, q, rc, rows, rpl, geo,
                               (lambda j, q=q: f'pf_{sid}_{q}_{rc}_{j}_', unsafe))
            o.append(f'{I}}}')

    def slot_dot(self, o, K3, q_c, wsrc, dt, vec, nv, lpp, pl, exact, rch, K, abase, geo):
        PB = geo['PB']
        o.append(f'{K3}float acc_[{PB}][{rch}];')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int j_ = 0; j_ < {PB}; ++j_)')
        o.append(f'{K3}  #pragma unroll')
        o.append(f'{K3}  for (int r_ = 0; r_ < {rch}; ++r_) acc_[j_][r_] = 0.0f;')
        self.mark(o, K3, 'stream dot start')
        o.append(f'{K3}#pragma unroll')
        o.append(f'{K3}for (int m_ = 0; m_ < {pl}; ++m_) {{')
        K4 = K3 + '  '
        o.append(f'{K4}const int kv_ = cl_ + m_ * {lpp};')
        if not exact:
            o.append(f'{K4}if (kv_ >= {nv}) break;')
        o.append(f'{K4}float wf_[{PB}][{vec}];')
        for j in range(PB):
            o.append(f'{K4}{self.vec_unpack(dt, vec, wsrc + f"[{j}][m_]", f"wf_[{j}]")}')
        o.append(f'{K4}#pragma unroll')
        o.append(f'{K4}for (int r_ = 0; r_ < {rch}; ++r_) {{')
        o.append(f'{K4}  const float* ar_ = sh_f + {abase} + r_ * {K} + kv_ * {vec};')
        o.append(f'{K4}  float av_[{vec}];')
        o.append(f'{K4}  {self.lds_vec_load(vec, "ar_", "av_")}')
        o.append(f'{K4}  #pragma unroll')
        o.append(f'{K4}  for (int j_ = 0; j_ < {PB}; ++j_)')
        o.append(f'{K4}    #pragma unroll')
        o.append(f'{K4}    for (int v_ = 0; v_ < {vec}; ++v_) acc_[j_][r_] = fmaf(av_[v_], wf_[j_][v_], acc_[j_][r_]);')
        o.append(f'{K4}}}')
        o.append(f'{K3}}}')
        if lpp > 1:
            o.append(f'{K3}#pragma unroll')
            o.append(f'{K3}for (int j_ = 0; j_ < {PB}; ++j_)')
            o.append(f'{K3}  #pragma unroll')
            o.append(f'{K3}  for (int r_ = 0; r_ < {rch}; ++r_) acc_[j_][r_] = group_red_sum(acc_[j_][r_], {lpp});')

    def slot_epilogue(self, s, c, st, fused, o, K3, q_c, rc, rows, rpl, geo, early):
        """After the butterfly every lane of a lane group holds the sums of
        all its (point, row) items; lane i of the group finishes items i,
        i + lpp, ... (``epi_item``). ``early``: (register prefix of round j,
        unsafe set) when the epilogue's early loads were issued at the barrier."""
        K5 = K3
        PB = geo['PB']
        for j in range(rpl):
            o.append(f'{K5}{{')
            K6 = K5 + '  '
            p_c, ok = self.epi_item(geo, q_c, j, rows, o, K6)
            o.append(f'{K6}const int p_ = {p_c};')
            o.append(f'{K6}if ({ok} && p_ < {geo["P"]}) {{')
            K7 = K6 + '  '
            self.decode('p_', st.pts, o, K7, prefix='ep_')
            if rows * PB == 1:
                val = 'acc_[0][0]'
            else:
                o.append(f'{K7}float av_ = acc_[0][0];')
                for it in range(1, rows * PB):
                    o.append(f'{K7}av_ = it_ == {it} ? acc_[{it // rows}][{it % rows}] : av_;')
                val = 'av_'
            lines = []
            if geo['reg']:
                self.decode(f'({rc * geo["rch"]} + r_)', geo['reg'], lines, K7, prefix='er_')
            if early is not None:
                self.capture = {'prefix': early[0](j), 'loads': [], 'unsafe': early[1]}
            try:
                self.epilogue(s, c, fused, self.epi_env(st, geo, rc), val, lines, K7)
            finally:
                self.capture = None
            o += lines
            o.append(f'{K6}}}')
            o.append(f'{K5}}}')

    # ------------------------------------------------------------ the other factor
    def direct_lds(self, c, reg):
        """LDS offset of the other factor when it is a private value laid out
        [reg axes, fold axes] and read at exactly those axes; else None."""
        A = c.A
        if A[0] != 'idx' or A[1] not in self.axes_of:
            return None
        r = self.root(A[1])
        if r not in self.private:
            return None
        want = list(reg) + list(c.fold_axes)
        if list(self.axes_of[r]) != want or list(A[2]) != [('name', a) for a in want]:
            return None
        return str(self.lds[r])

    def stage_A(self, c, reg, rc, rch, R, K, abase, o, I):
        """The other factor at every (row, fold point) of this row chunk into
        LDS [row, fold] (rows past R are zero). A value of global scratch laid
        out [reg axes, fold axes] is copied with 16-byte coherent loads;
        anything else is evaluated point by point, all loads of a thread issued
        before its LDS stores."""
        A = c.A
        o.append(f'{I}vh_lds_sync();')
        want = list(reg) + list(c.fold_axes)
        if (A[0] == 'idx' and A[1] in self.axes_of and self.root(A[1]) in self.g
                and self.root(A[1]) not in self.private and self.root(A[1]) not in self.fx
                and self.root(A[1]) not in self.peel_active
                and list(self.axes_of[self.root(A[1])]) == want
                and list(A[2]) == [('name', a) for a in want] and K % 4 == 0):
            rows = min(rch, R - rc * rch)
            off = self.g[self.root(A[1])] + rc * rch * K
            o.append(f'{I}stage_ldc4(sh_f + {abase}, rb_S, {off}, {rows * K});  // stage {A[1]}')
            if rows < rch:
                o.append(f'{I}for (int e_ = tid; e_ < {(rch - rows) * K}; e_ += {self.BLOCK}) '
                         f'sh_f[{abase} + {rows * K} + e_] = 0.0f;')
            o.append(f'{I}vh_lds_sync();')
            return
        T = -(-(rch * K) // self.BLOCK)
        o.append(f'{I}#pragma unroll' + ('' if T <= 16 else ' 8'))
        o.append(f'{I}for (int it_ = 0; it_ < {T}; ++it_) {{')
        J2 = I + '  '
        o.append(f'{J2}const int e_ = tid + it_ * {self.BLOCK};')
        o.append(f'{J2}if (e_ < {rch * K}) {{')
        J3 = J2 + '  '
        o.append(f'{J3}const int ar_ = e_ / {K}, ak_ = e_ % {K};')
        env = self.decode('ak_', c.fold_axes, o, J3, prefix='fa_')
        o.append(f'{J3}float v_ = 0.0f;')
        o.append(f'{J3}if ({rc * rch} + ar_ < {R}) {{')
        if reg:
            env.update(self.decode(f'({rc * rch} + ar_)', reg, o, J3 + '  ', prefix='ra_'))
        pre = []
        v, t = self.expr(c.A, env, pre, J3 + '  ')
        o += pre
        o.append(f'{J3}  v_ = {self.as_float(v, t)};')
        o.append(f'{J3}}}')
        o.append(f'{J3}sh_f[{abase} + e_] = v_;')
        o.append(f'{J2}}}')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')

    # ------------------------------------------------------------ small helpers
    def load_type(self, dt, vec):
        if dt == 'f16':
            return {8: 'vh_u32x4', 4: 'vh_u32x2', 2: 'unsigned', 1: 'vh_half'}[vec]
        return {4: 'vh_f32x4', 2: 'vh_f32x2', 1: 'float'}[vec]

    def weights_kept(self, kind, src=None):
        """Load a stream's weights with the temporal cache policy (else
        nontemporal)? Measured on the MI355X (GPT-2 small): below 4 rows every
        weight stream (B=1 step 230 -> 221 us); from 4 rows the streams outside
        the layer loop (the output head, read once a step), the streams whose
        fold is split over blocks (B=8 327 -> 312 us) and the attention
        out-projection when its copies over all layers are small (B=8
        320 -> 311 us); keeping the other layer weights too was slower: the
        cache then holds neither."""
        if self.batch < 4:
            return True
        if kind == 'proj' and src is not None:
            return 2 * math.prod(self.res[src][0]) <= PROJ_KEPT_BYTES
        return kind == 'split' or not self.loops

    def w16(self, kind, src=None):
        """The 16-byte weight load function for a stream of ``kind`` (over residue ``src``)."""
        return 'ldg16_t' if self.weights_kept(kind, src) else 'ldg16_nt'

    def nt_load(self, dt, vec, rr, idx, kept=False):
        """Streamed load of ``vec`` elements at element index ``idx`` through descriptor ``rr``."""
        if dt == 'f16' and vec == 8 and kept:
            return f'ldg16_t({rr}, {idx})'
        if dt == 'f16':
            return {8: f'ldg16_nt({rr}, {idx})', 4: f'ldg8_nt({rr}, {idx})', 2: f'ldg4_nt({rr}, {idx})',
                    1: f'(vh_half)(ldg4_nt({rr}, {idx}) & 0xffffu)'}[vec]
        return {4: f'__builtin_bit_cast(vh_f32x4, ldg16_nt({rr}, 2u * ({idx})))',
                2: f'__builtin_bit_cast(vh_f32x2, ldg8_nt({rr}, 2u * ({idx})))',
                1: f'ldg_f({rr}, {idx})'}[vec]

    def lds_vec_load(self, vec, ptr, dst):
        if vec == 8:
            return (f'{{ const vh_f32x4 x0_ = *(const vh_f32x4*)({ptr}), x1_ = *(const vh_f32x4*)({ptr} + 4); '
                    f'{dst}[0] = x0_.x; {dst}[1] = x0_.y; {dst}[2] = x0_.z; {dst}[3] = x0_.w; '
                    f'{dst}[4] = x1_.x; {dst}[5] = x1_.y; {dst}[6] = x1_.z; {dst}[7] = x1_.w; }}')
        if vec == 4:
            return (f'{{ const vh_f32x4 x0_ = *(const vh_f32x4*)({ptr}); '
                    f'{dst}[0] = x0_.x; {dst}[1] = x0_.y; {dst}[2] = x0_.z; {dst}[3] = x0_.w; }}')
        if vec == 2:
            return f'{{ const vh_f32x2 x0_ = *(const vh_f32x2*)({ptr}); {dst}[0] = x0_.x; {dst}[1] = x0_.y; }}'
        return f'{dst}[0] = {ptr}[0];'
