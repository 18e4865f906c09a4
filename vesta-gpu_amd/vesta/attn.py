"""Attention groups: scores, softmax statistics and weighted values of one
leading point (a batch row and head) in one block, K/V rows in registers.

The pattern (what ``gpt2.vst`` Q5-Q7 lower to after hoisting and inlining):

    sc[L.., s] = EPI1(fold sum e: A1[L.., e] * K[.., s, .., e])     lane contraction over a cache
    mx[L..]    = fold max s: sc[L.., s]
    hs[L..]    = fold sum s: F(sc[L.., s], mx[L..])
    o[L.., e]  = EPI4(fold sum s: A4(sc, mx, hs)[L.., s] * V[.., s, .., e])

with ``s`` the dynamic context axis and K, V residues the step emits into.
Each compute wave lane owns one (position, 8-element chunk of e) pair per
slot, the same pair for K and for V, so a lane's K and V loads are 16 bytes
each and a position's score is a butterfly over its lanes. Rows of the
cache written by earlier steps are loaded at the barrier before the group
(between grid_arrive and grid_wait) into registers; only the row the step
itself emits, and the query, are read after the wait. The statistics are
block reductions; the weighted values are reduced over positions inside a
wave and then across waves through LDS.

Numerics follow the program statement by statement: the score epilogue,
``F`` and ``A4`` are evaluated per position exactly as written (so the
weight is ``exp(sc - mx) / hs`` per position, as in the program); only the
order of the sums over ``s`` and ``e`` differs from a sequential sum.
"""
from __future__ import annotations

import math


ATTN_PREFETCH_SLOTS = 8      # cache rows per lane issued early (K and V each)
ATTN_CHUNK = 4               # longer contexts: slots per chunk of the running (online) softmax
ATTN_CHUNK_LOOP = 3          # from this many chunks, a run-time loop over two chunks' registers (unrolled,
                             # the long chunk sequence spilled: GPT-2 small with a 1024-position cache)
ATTN_ONLINE_SHORT = True     # shorter ones: the running softmax too, as one chunk of every slot (no block-wide
                             # maximum and sum)
PROJ_MIN_REPLICAS = 2        # fuse the out-projection only if every leading point gets this many blocks
PROJ_EARLY_SLOTS = 8         # projection weights issued at the barrier when a lane needs at most this many loads
READY_ATTN = False           # attention waits for the blocks that made its rows (readiness flags) instead of
                             # a grid barrier, its projection's sum in two layer buffers: two grid barriers
                             # per GPT-2 layer, but slower (same box: B=8 306-312 us per step against 299,
                             # B=1 212-218 against 205-208, equal tokens and logits), so off
                             # (B=8: 7 loads; early, with the prefetch budget cut to fit, 316 -> 307 us per step)


class AttnMixin:
    def attn_of(self, lead, members):
        """Pattern description of an attention group, or None."""
        if len(members) != 4:
            return None
        t1, t2, t3, t4 = members
        local = set(self.group_local.get(id(t1), []))
        if local != {t1[1], t2[1], t3[1]}:
            return None
        c1, c4 = self.contraction(t1), self.contraction(t4)
        if c1 is None or c4 is None or c1.kind != 'lane' or c4.kind != 'tile':
            return None
        if c1.W not in self.emitted or c4.W not in self.emitted or c1.reg_axes or c4.reg_axes:
            return None
        if self.res[c1.W][1] != 'f16' or self.res[c4.W][1] != 'f16':
            return None
        plen = len(lead)
        if list(t1[2][:plen]) != list(lead) or len(t1[2]) != plen + 1:
            return None
        S = t1[2][-1]
        if S not in self.dynamic or len(c1.fold_axes) != 1:
            return None
        E1 = c1.fold_axes[0]
        same = [('name', a) for a in list(lead) + [S]]
        at_lead = [('name', a) for a in lead]
        e2 = t2[3]
        if list(t2[2]) != list(lead) or e2 != ('fold', 'max', S, ('idx', t1[1], same)):
            return None
        e3 = t3[3]
        if list(t3[2]) != list(lead) or e3[0] != 'fold' or e3[1] != 'sum' or e3[2] != S:
            return None
        if not self._reads_at(e3[3], {t1[1]: same, t2[1]: at_lead}):
            return None
        if list(t4[2]) != list(lead) + [c4.contig] or c4.fold_axes != [S]:
            return None
        if not self._reads_at(c4.A, {t1[1]: same, t2[1]: at_lead, t3[1]: at_lead}):
            return None
        E4 = c4.contig
        nE1, nE4 = self.static[E1], self.static[E4]
        if nE1 % 8 or nE4 % 8 or 64 % (nE1 // 8) or 64 % (nE4 // 8) or nE1 != nE4:
            return None
        # both caches read as W[.., s, .., e] with e their last axis; the step's own row
        # is the one its emits write
        rows = []
        for W in (c1.W, c4.W):
            emits = [x for x in self.emit_stmts if x[1] == W]
            if len(emits) != 1:
                return None
            widx = c1.widx if W == c1.W else c4.widx
            pos = [i for i, x in enumerate(widx) if x == ('name', S)]
            if len(pos) != 1:
                return None
            erow = emits[0][2][pos[0]]
            if self.free_axes(erow) - set(lead) - self.steps:
                return None
            rows.append(erow)
        if rows[0] != rows[1]:
            return None
        return dict(t=members, c1=c1, c4=c4, S=S, E=E1, E4=E4, nE=nE1, erow=rows[0], lead=list(lead))

    # ------------------------------------------------------------ projection
    def find_projections(self, ss):
        """Attention groups that also do the contraction reading their output
        (the out-projection): see ``proj_of``. The contraction and the
        statement adding it to a residual are then made by the group's blocks."""
        for i, s in enumerate(ss):
            if s[0] == 'step':
                self.find_projections(s[6])
                continue
            if id(s) not in self.groups:
                continue
            lead, members = self.groups[id(s)]
            at = self.attn_of(lead, members)
            j = i + len(members)
            if at is None or j + 1 >= len(ss):
                continue
            pj = self.proj_of(at, ss[j], ss[j + 1])
            if pj is None:
                continue
            self.proj[id(s)] = pj
            self.elided |= {id(ss[j]), id(ss[j + 1])}
            self.elided_vals |= {ss[j][1], members[3][1]}
            self.fx.add(ss[j + 1][1])

    def proj_of(self, at, so, sz):
        """The pattern

            oo[P.., d] = fold sum F..: fold sum e: o[L.., e] * W[.., F.. e .., d]
            z1[P.., d] = BASE + oo[P.., d]          (oo added, nothing else done to it)

        right after attention group ``at`` (output o[L.., e]), where each
        leading axis of o is a point axis P or a fold axis F of oo, W is an
        fp16 residue streamed through its transposed copy, and o and oo have no
        other readers. The blocks of a leading point then multiply its 64-ish
        outputs by their slice of W (rows of the transposed copy, split over
        ``R`` replica blocks that each redo the point's attention) and add the
        products into z1, kept as a 64-bit fixed-point sum (exact, so the order
        of the adds does not change the result); BASE is stored into z1 in the
        phase before the attention. Returns the description, or None."""
        t4 = at['t'][3]
        o, lead = t4[1], at['lead']
        if so[0] != 'let' or sz[0] != 'let' or self.place.get(id(so)) != 'tile':
            return None
        c = self.info[id(so)]
        oo, z1 = so[1], sz[1]
        if c.epi != ('name', '__acc') or c.pt_axes or self.res[c.W][1] != 'f16':
            return None
        carries = set(self.alias) | set(self.alias.values())
        for n in (o, oo, z1):
            if n in self.outputs or n in carries or self.root(n) != n:
                return None
        if self.readers_of.get(o, set()) != {id(so)} or self.readers_of.get(oo, set()) != {id(sz)}:
            return None
        A = c.A
        if A[0] != 'idx' or A[1] != o or any(x[0] != 'name' for x in A[2]):
            return None
        names = [x[1] for x in A[2]]
        fold = list(c.fold_axes)
        plen = len(lead)
        if len(names) != plen + 1 or names[-1] != fold[-1] or len(set(names)) != len(names):
            return None
        if set(fold) - set(names) or self.static[names[-1]] != at['nE']:
            return None
        pmap, fmap = {}, {}
        for k in range(plen):
            n = names[k]
            if self.static.get(n) != self.static[lead[k]]:
                return None
            if n in fold:
                fmap[n] = k
            elif n in so[2] and n != c.contig:
                pmap[n] = k
            else:
                return None
        if set(so[2]) != set(pmap) | {c.contig} or list(sz[2]) != list(so[2]):
            return None
        target = ('idx', oo, [('name', a) for a in so[2]])
        if not self._additive(sz[3], target, oo):
            return None
        base = self.rebuild_expr(sz[3], lambda n: ('num', 0.0) if n == target else n)
        if self.reads(base) & {t[1] for t in at['t']}:
            return None
        st = self.stream_of(c)
        if st is None or st.pack is None or st.vec != 8:
            return None
        G = self.size(lead)
        R = self.grid // G
        if R < PROJ_MIN_REPLICAS:
            if self.grid_wide // G >= PROJ_MIN_REPLICAS:
                self.proj_wider = True
            return None
        # fold position of (F.., e): the flat index over the fold axes, last fastest
        strides, acc = {}, 1
        for a in reversed(fold):
            strides[a] = acc
            acc *= self.static[a]
        D = self.static[c.contig]
        return dict(so=so, sz=sz, c=c, st=st, base=base, pmap=pmap, fmap=fmap, strides=strides,
                    R=R, D=D, DPR=-(-D // R))

    def _additive(self, e, target, name):
        """Is e = (something) + target, target read once and only through + and
        the left side of -?"""
        hits = [n for n in self.nodes_of(e) if n[0] in ('idx', 'name') and n[1] == name]
        if hits != [target]:
            return False

        def walk(x):
            if x == target:
                return True
            if x[0] == 'bin' and x[1] == '+':
                return walk(x[2]) or walk(x[3])
            if x[0] == 'bin' and x[1] == '-':
                return walk(x[2])
            return False
        return walk(e)

    def gen_proj_base(self, pj, out, ind):
        """z1 = BASE at every point, spread over all blocks (a few threads
        each), unless a private run before did it (by atomic adds when the
        group waits on readiness flags: other blocks' projections may be in
        already)."""
        sz = pj['sz']
        if pj.get('base_done'):
            return
        if pj.get('ready') is not None:
            self.chain_base(pj, out, ind)
            return
        self.emit_base(sz, sz[1], list(sz[2]), pj['base'], out, ind, sync=True)

    # ------------------------------------------------------------ readiness flags
    def find_ready_attn(self, ss, step=None):
        """Attention groups with a projection whose dirty inputs all come from
        the stream right before them (its values, and cache rows its fused
        emits store): the group's blocks then wait for the blocks that made
        their rows instead of a grid barrier (``attn_ready``). The projection's
        fixed-point sum is then kept in two buffers by layer parity: a layer's
        adds go into one while the other, read by the layer before, is
        cleared for the next."""
        if not READY_ATTN:
            return
        for i, s in enumerate(ss):
            if s[0] == 'step':
                self.find_ready_attn(s[6], s)
                continue
            pj = self.proj.get(id(s))
            if pj is None or step is None:
                continue
            lead, members = self.groups[id(s)]
            rd = self.attn_ready(ss, i, self.attn_of(lead, members), pj)
            if rd is None:
                continue
            z1 = self.root(pj['sz'][1])
            if z1 in self.fx_copies or z1 in self.fx_parity:
                continue
            pj.update(ready=rd, p2p=True, z=z1, axes=list(pj['sz'][2]))
            var = step[3]
            self.fx_parity[z1] = (f'l_{var}', var, self.static[var], 'layer')
            # the loop's carry, added into by a local fold or a split in the same
            # body, can no longer be cleared in the phase before theirs (it is read
            # there now): it alternates between two buffers as well
            ids = {id(t) for t in step[6]}
            for sid_, sk in list(self.chains.items()) + list(self.splits.items()):
                if sid_ in ids and (sk is not None and (sid_ in self.chains or sk.get('p2p'))):
                    self.fx_parity[sk['z']] = (f'l_{var}', var, self.static[var], 'carry')

    def attn_ready(self, ss, i, at, pj):
        """The producers of group ``at`` (statement ss[i]): the stream u before
        it and the emits fused into u between them. Returns (u, points per
        block of u, [(const, {axis: coef}), ..]: u's point index of each read
        the group makes of u's values or of the rows the emits store, affine in
        the group's leading axes and free axes), or None."""
        j, emits = i - 1, {}
        while j >= 0 and ss[j][0] == 'emit':
            emits[ss[j][1]] = ss[j]
            j -= 1
        if j < 0 or ss[j][0] != 'let':
            return None
        u = ss[j]
        if self.place.get(id(u)) not in ('tile', 'lane') or id(u) in self.splits or id(u) in self.groups:
            return None
        cu = self.info.get(id(u))
        st = self.stream_of(cu) if getattr(cu, 'kind', None) in ('tile', 'lane') else None
        if st is None or len(st.pts) != 1:
            return None
        U, reg = self.root(u[1]), list(cu.reg_axes)
        if list(u[2]) != reg + list(st.pts) or any(a not in at['lead'] for a in reg):
            return None
        deps = []

        def u_index(n):
            if list(n[2][:len(reg)]) != [('name', a) for a in reg]:
                return None
            return self.affine(n[2][-1])
        for t in at['t']:
            for n in self.nodes_of(t[3]):
                if n[0] != 'idx':
                    continue
                if n[1] in self.axes_of and self.root(n[1]) == U:
                    aff = u_index(n)
                elif n[1] in emits:
                    e = emits[n[1]]
                    # the emit's row index must name the group's leading axes where the read does
                    if len(e[2]) != len(n[2]) or any(x[0] == 'name' and x[1] in at['lead'] and y != x
                                                     for x, y in zip(n[2], e[2])):
                        return None
                    vals = [m for m in self.nodes_of(e[3]) if m[0] == 'idx' and m[1] in self.axes_of
                            and self.root(m[1]) == U]
                    aff = u_index(vals[0]) if len(vals) == 1 else None
                else:
                    continue
                if aff is None or any(a not in self.static for a in aff[1]):
                    return None
                if aff not in deps:
                    deps.append(aff)
        if not deps:
            return None
        P = self.size(st.pts)
        PPB = -(-P // self.grid)
        lead = at['lead']
        # at most 64 producers per consumer, over every leading point
        ext = [self.static[a] for a in lead]
        for flat in range(math.prod(ext)):
            vals, r = {}, flat
            for a, n in zip(reversed(lead), reversed(ext)):
                vals[a] = r % n
                r //= n
            total = 0
            for const, coefs in deps:
                lo, hi = self.dep_range(const, coefs, vals)
                total += hi // PPB - lo // PPB + 1
            if total > 64:
                return None
        return dict(u=u, U=U, PPB=PPB, deps=deps, emits=set(emits))

    def attn_ready_point(self, at, pj, rd, reads, writes, out, ind):
        """In place of the grid barrier before the group: the next layer's
        buffer of the projection's sum is cleared, then every block publishes
        and the group's blocks wait for the makers of their rows."""
        from .chain import ChainError
        t1, lead = at['t'][0], at['lead']
        z1 = pj['z']
        if (reads - {rd['U']} - rd['emits']) & self.dirty or (writes - {z1}) & (self.readers | self.dirty) \
                or z1 in self.readers:
            raise ChainError(f'attention {t1[1]}: its phase would need a barrier after all')
        n4 = self.fx_words(z1) // 4
        self.trace.append(('clear', z1, None, 1))
        out.append(f'{ind}for (int e_ = (int)blockIdx.x + (int)nblk * tid; e_ < {n4}; e_ += nthr) '
                   f'stz4(rb_S, {self.gofs(z1, ahead=1)} + 4u * (unsigned)e_);  // clear the next layer\'s {z1}')
        G = self.size(lead)
        setup = []
        env = self.decode(f'((int)blockIdx.x % {G})', lead, setup, '', prefix='rl_')
        vals = {a: env[a][0] for a in lead}
        PPB = rd['PPB']
        ranges = []
        for const, coefs in rd['deps']:
            lo, hi = self.dep_range(const, coefs, vals)
            ranges.append((f'({lo}) / {PPB}', f'({hi}) / {PPB}'))
        self.trace.append(('flags', t1[1], frozenset({rd['U']} | set(rd['emits']))))
        self.trace.append(('flagrange', 'attention', ranges, f'(int)blockIdx.x < {G * pj["R"]}', tuple(setup),
                           dict(lead=list(lead), ext=[self.static[a] for a in lead], G=G, PPB=PPB, deps=rd['deps'],
                                free={a: self.static[a] for _, co in rd['deps'] for a in co if a not in lead},
                                grid=self.grid)))
        self.ready_point(t1[1], ranges, f'(int)blockIdx.x < {G * pj["R"]}', out, ind, rd['u'][1], setup)

    def dep_range(self, const, coefs, lead_vals):
        """(lowest, highest) point of an affine index with the leading axes
        given (all numbers, or all C expressions) and every other axis over
        its extent."""
        num = all(isinstance(v, int) for v in lead_vals.values())
        lo, hi = [const], [const]
        for a, k in coefs.items():
            if a in lead_vals:
                term = k * lead_vals[a] if num else f'{k} * ({lead_vals[a]})'
                lo.append(term)
                hi.append(term)
            else:
                span = k * (self.static[a] - 1)
                (lo if span < 0 else hi).append(span)
        if num:
            return sum(lo), sum(hi)
        return ' + '.join(map(str, lo)), ' + '.join(map(str, hi))

    def _reads_at(self, e, allowed):
        """Does e read group values only at the given index lists (and no folds)?"""
        for n in self.nodes_of(e):
            if n[0] == 'fold':
                return False
            if n[0] == 'idx' and n[1] in allowed and list(n[2]) != allowed[n[1]]:
                return False
            if n[0] == 'name' and n[1] in allowed:
                return False
        return True

    # ------------------------------------------------------------ codegen
    def gen_attn(self, at, out, ind, pj=None):
        """The group's code; with ``pj`` (see ``proj_of``) also the projection
        of its output, added into a fixed-point sum."""
        t1, t2, t3, t4 = at['t']
        c1, c4, S, lead = at['c1'], at['c4'], at['S'], at['lead']
        if pj is not None:
            self.gen_proj_base(pj, out, ind)
        names = {t[1] for t in at['t']}
        local = self.group_local.get(id(t1), [])
        reads = self.root_reads([t[3] for t in at['t']], exclude=names)
        writes = {self.root(t[1]) for t in at['t'] if t[1] not in local}
        if pj is not None:
            writes = (writes - {t4[1]}) | {pj['sz'][1]}
        rd = pj.get('ready') if pj is not None else None
        if rd is not None:
            self.attn_ready_point(at, pj, rd, reads, writes, out, ind)
        else:
            self.sync(reads, writes, out, ind, t1[1])
        for t in at['t']:
            self.plan.append((self.show_stmt(t), f'attention[{", ".join(lead)}]'))
        if pj is not None:
            self.plan.append((self.show_stmt(pj['so']), f'attention[{", ".join(lead)}] projection x{pj["R"]}'))
        nE = at['nE']
        LPE = nE // 8                      # lanes per position (16-byte chunks of e)
        PPW = 64 // LPE                    # positions per wave per slot
        NW = self.NWAVE - 1                # compute waves (the last wave polls barriers)
        PPP = NW * PPW                     # positions per block per slot
        smax = self.static[S]
        NPS = -(-smax // PPP)
        NPF = min(NPS, ATTN_PREFETCH_SLOTS, self.pf_budget // 8)
        # more slots than registers hold: the softmax runs over chunks of slots
        # (running maximum and sum, rescaled), the rows of the next chunk in
        # flight while a chunk is used
        online = (NPS > ATTN_PREFETCH_SLOTS or ATTN_ONLINE_SHORT) and self._softmax_form(at)
        chunk = ATTN_CHUNK if NPS > ATTN_PREFETCH_SLOTS else NPS
        if online:
            NPF = min(NPF, chunk)               # the first chunk at the barrier, the rest streamed
        G = self.size(lead)
        R = pj['R'] if pj is not None else 1      # blocks per leading point (each redoes its attention)
        GR = G * R
        sid = self.fresh('a')
        kq, vq = f'kq_{sid}', f'vq_{sid}'
        T = self.ext_c(S)
        rbK, rbV = f'rb_{c1.W}', f'rb_{c4.W}'
        self.red_floats = max(getattr(self, 'red_floats', 4), 2 * self.NWAVE)
        red_o = self.lds_floats + self.stage_top
        self.stage_floats = max(self.stage_floats, self.stage_top + NW * nE)

        def row_index(W, c, env):
            """Element index of (s, e-chunk start) in cache W: lines, expression."""
            lines = []
            ix = [self.index(x, env, lines, '') for x in c.widx]
            return lines, self.addr(ix, self.res_strides(W))

        def slot_env(k, lead_env):
            env = dict(lead_env)
            env[S] = (f's{k}_', 'int')
            return env

        def erow_c(lead_env):
            lines = []
            v = self.index(at['erow'], lead_env, lines, '')
            return lines, v

        def load_kv(k, lead_env, early):
            """Lines loading K and V of slot k into kq[k], vq[k] (zeros where the
            position is out of range; early: only rows other than the step's own)."""
            lines = [f'{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;']
            el, ev = erow_c(lead_env)
            lines += el
            cond = f'wave < {NW} && s{k}_ < {T}' + (f' && s{k}_ != ({ev})' if early else '')
            env = slot_env(k, lead_env)
            env[at['E']] = ('(cl_ * 8)', 'int')
            l1, a1 = row_index(c1.W, c1, env)
            env4 = slot_env(k, lead_env)
            env4[at['E4']] = ('(cl_ * 8)', 'int')
            l4, a4 = row_index(c4.W, c4, env4)
            lines.append(f'  if ({cond}) {{')
            lines += ['    ' + x for x in l1 + l4]
            lines.append(f'    {kq}[{k}] = ldc16_h({rbK}, {a1});')
            lines.append(f'    {vq}[{k}] = ldc16_h({rbV}, {a4});')
            lines.append('  }' + ('' if early else ' else { ' + f'{kq}[{k}] = vh_u32x4{{0u, 0u, 0u, 0u}}; '
                                                     f'{vq}[{k}] = vh_u32x4{{0u, 0u, 0u, 0u}}; }}'))
            lines.append('}')
            return lines

        def load_kv_at(tag, slot, lead_env, kd, vd):
            """Lines loading K and V of the slot at C expression ``slot`` into
            kd, vd (zeros where the position is out of range)."""
            lines = [f'{{ const int s{tag}_ = ({slot}) * {PPP} + wave * {PPW} + sub_;']
            env = slot_env(tag, lead_env)
            env[at['E']] = ('(cl_ * 8)', 'int')
            l1, a1 = row_index(c1.W, c1, env)
            env4 = slot_env(tag, lead_env)
            env4[at['E4']] = ('(cl_ * 8)', 'int')
            l4, a4 = row_index(c4.W, c4, env4)
            lines.append(f'  if (wave < {NW} && s{tag}_ < {T}) {{')
            lines += ['    ' + x for x in l1 + l4]
            lines.append(f'    {kd} = ldc16_h({rbK}, {a1});')
            lines.append(f'    {vd} = ldc16_h({rbV}, {a4});')
            lines.append(f'  }} else {{ {kd} = vh_u32x4{{0u, 0u, 0u, 0u}}; {vd} = vh_u32x4{{0u, 0u, 0u, 0u}}; }}')
            lines.append('}')
            return lines

        lane_decl = f'const int sub_ = lane / {LPE}, cl_ = lane % {LPE};'
        self.decls.append(f'vh_u32x4 {kq}[{NPS}];')
        self.decls.append(f'vh_u32x4 {vq}[{NPS}];')

        def lead_lines(gp):
            lines = []
            env = self.decode(gp, lead, lines, '', prefix='al_')
            return lines, env

        if pj is not None:
            c5, st5 = pj['c'], pj['st']
            DPR, D = pj['DPR'], pj['D']
            NQP = -(-DPR // (NW * PPW))               # projection rounds: PPW rows per wave each
            early = NQP <= PROJ_EARLY_SLOTS
            wp = f'wp_{sid}'
            if early:
                self.decls.append(f'vh_u32x4 {wp}[{NQP}];')

        def proj_loads(lenv, rp):
            """Lines loading this lane's 8 weights of each projection round
            (row d of the transposed copy, the point's fold positions)."""
            lines = []
            foff = ' + '.join(f'{pj["strides"][a]} * {lenv[lead[k]][0]}' for a, k in pj['fmap'].items()) or '0'
            rs = self.res_strides(st5.src)
            for q in range(NQP):
                lines.append(f'{{ const int dl_ = {q * NW * PPW} + wave * {PPW} + sub_, d_ = {rp} * {DPR} + dl_;')
                lines.append(f'  if (wave < {NW} && dl_ < {DPR} && d_ < {D}) {{')
                pre = []
                ix = [self.index(x, {c5.contig: ('d_', 'int')}, pre, '    ') for x in st5.prefix_idx]
                lines += pre
                lines.append(f'    {wp}[{q}] = {self.w16("proj", st5.src)}({self.rsrc(st5.src)}, (unsigned)({self.addr(ix, rs[:-1])}) + '
                             f'{st5.c0}u + (unsigned)({foff}) + (unsigned)cl_ * 8u);')
                lines.append(f'  }} else {wp}[{q}] = vh_u32x4{{0u, 0u, 0u, 0u}};')
                lines.append('}')
            return lines

        def make(step_override):
            saved = self.override_step(step_override)
            try:
                ll, lenv = lead_lines(f'((int)blockIdx.x % {G})' if R > 1 else '(int)blockIdx.x')
                lines = [f'if ((int)blockIdx.x < {GR}) {{', '  ' + lane_decl] + ['  ' + x for x in ll]
                for k in range(NPF):
                    lines += ['  ' + x for x in load_kv(k, lenv, True)]
                if pj is not None and early:
                    lines += ['  ' + x for x in proj_loads(lenv, f'((int)blockIdx.x / {G})')]
                return lines + ['}']
            finally:
                self.restore_step(saved)
        self.place_prefetch(make, out, ind)

        o = out
        I = ind + '  '
        # one point per block when there are blocks enough: then every block's
        # point is its first, whose rows were loaded early
        once = GR <= self.grid
        head = (f'{{ const int gi_ = blockIdx.x; if (gi_ < {GR}) {{' if once else
                f'for (int gi_ = blockIdx.x; gi_ < {GR}; gi_ += nblk) {{')
        o.append(f'{ind}{head}  // attention {t1[1]}..{t4[1]}: '
                 f'{LPE} lanes/position, {PPP} positions/slot, {NPS} slots, {NPF} loaded early'
                 + (f', {R} blocks per point' if R > 1 else ''))
        o.append(f'{I}{lane_decl}')
        o.append(f'{I}const int gp_ = gi_ % {G}, rp_ = gi_ / {G};' if R > 1 else f'{I}const int gp_ = gi_;')
        ll, lenv = lead_lines('gp_')
        o += [I + x for x in ll]
        o.append(f'{I}const bool first_ = ' + ('true;' if once else 'gi_ == (int)blockIdx.x;'))
        # the step's own row (and every row when this is not the block's first point)
        el, ev = erow_c(lenv)
        o += [I + x for x in el]
        for k in range(NPF if online else NPS):
            o.append(f'{I}{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;')
            if k < NPF:
                o.append(f'{I}  if (!first_ || s{k}_ == ({ev}) || s{k}_ >= {T}) {{')
            else:
                o.append(f'{I}  {{')
            o += [I + '    ' + x for x in load_kv(k, lenv, False)]
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        if pj is not None and not early:
            o.append(f'{I}vh_u32x4 {wp}[{NQP}];')
        elif pj is not None:
            # a block's later points (none when every point has its own blocks) load here
            o.append(f'{I}if (!first_) {{')
            o += [I + '  ' + x for x in proj_loads(lenv, 'rp_')]
            o.append(f'{I}}}')
        self.mark(o, I, 'attention: rows')
        # the query chunk of this lane
        o.append(f'{I}float qv_[8];')
        o.append(f'{I}#pragma unroll')
        o.append(f'{I}for (int v_ = 0; v_ < 8; ++v_) {{')
        qenv = dict(lenv)
        qenv[at['E']] = ('(cl_ * 8 + v_)', 'int')
        pre = []
        qv, qt = self.expr(c1.A, qenv, pre, I + '  ')
        o += pre
        o.append(f'{I}  qv_[v_] = {self.as_float(qv, qt)};')
        o.append(f'{I}}}')
        if online:
            self.attn_online(at, o, I, lenv, NPS, NPF, PPP, PPW, LPE, NW, T, nE, kq, vq, slot_env, load_kv,
                             red_o, pj, po_ref := [], chunk, load_kv_at)
            po = po_ref[0]
            if pj is not None:
                if not early:
                    o += [I + x for x in proj_loads(lenv, 'rp_')]
                self.gen_proj_tail(pj, lenv, lead, po, wp, NQP, NW, PPW, LPE, o, I)
            o.append(f'{ind}}}' + ('}' if once else ''))
            self.note(reads, writes)
            self.mark(out, ind, f'attention {t1[1]}..{t4[1]}')
            return
        # scores
        o.append(f'{I}float sk_[{NPS}];')
        o.append(f'{I}float mloc_ = -INFINITY;')
        for k in range(NPS):
            o.append(f'{I}{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;')
            o.append(f'{I}  float wf_[8];')
            o.append(f'{I}  unpack8({kq}[{k}], wf_);')
            o.append(f'{I}  float d_ = 0.0f;')
            o.append(f'{I}  #pragma unroll')
            o.append(f'{I}  for (int v_ = 0; v_ < 8; ++v_) d_ = fmaf(qv_[v_], wf_[v_], d_);')
            o.append(f'{I}  d_ = group_red_sum(d_, {LPE});')
            venv = dict(slot_env(k, lenv))
            venv['__acc'] = ('d_', 'float')
            pre = []
            sv, st_ = self.expr(c1.epi, venv, pre, I + '  ')
            o += pre
            o.append(f'{I}  sk_[{k}] = (wave < {NW} && s{k}_ < {T}) ? {self.as_float(sv, st_)} : -INFINITY;')
            o.append(f'{I}  mloc_ = fmaxf(mloc_, sk_[{k}]);')
            o.append(f'{I}}}')
        self.mark(o, I, 'attention: scores')
        if pj is not None and not early:
            # issued once the keys are dead (their registers take these) and after
            # the cache rows, so waiting for the values does not wait for these
            o += [I + x for x in proj_loads(lenv, 'rp_')]
        o.append(f'{I}const float mx_ = block_red_max(mloc_, red_sh);')
        self.mark(o, I, 'attention: max')
        # the softmax denominator: each position once (its lane group's first lane)
        o.append(f'{I}float hloc_ = 0.0f;')
        for k in range(NPS):
            o.append(f'{I}{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;')
            fe, fx = self._subst(t3[3][3], {t1[1]: f'sk_[{k}]', t2[1]: 'mx_'})
            pre = []
            fv, ft = self.expr(fe, {**slot_env(k, lenv), **fx}, pre, I + '  ')
            o += pre
            o.append(f'{I}  if (cl_ == 0 && wave < {NW} && s{k}_ < {T}) hloc_ += {self.as_float(fv, ft)};')
            o.append(f'{I}}}')
        o.append(f'{I}const float hs_ = block_red_sum(hloc_, red_sh);')
        self.mark(o, I, 'attention: sum')
        # weighted values
        o.append(f'{I}float ov_[8];')
        o.append(f'{I}#pragma unroll')
        o.append(f'{I}for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = 0.0f;')
        for k in range(NPS):
            o.append(f'{I}{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;')
            o.append(f'{I}  if (wave < {NW} && s{k}_ < {T}) {{')
            ae, ax = self._subst(c4.A, {t1[1]: f'sk_[{k}]', t2[1]: 'mx_', t3[1]: 'hs_'})
            pre = []
            av, aty = self.expr(ae, {**slot_env(k, lenv), **ax}, pre, I + '    ')
            o += pre
            o.append(f'{I}    const float w_ = {self.as_float(av, aty)};')
            o.append(f'{I}    float wf_[8];')
            o.append(f'{I}    unpack8({vq}[{k}], wf_);')
            o.append(f'{I}    #pragma unroll')
            o.append(f'{I}    for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = fmaf(w_, wf_[v_], ov_[v_]);')
            o.append(f'{I}  }}')
            o.append(f'{I}}}')
        self.mark(o, I, 'attention: pv')
        if PPW > 1:
            o.append(f'{I}#pragma unroll')
            o.append(f'{I}for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = wave_red_sum_hi(ov_[v_], {LPE});')
        o.append(f'{I}if (wave < {NW} && sub_ == 0) {{')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int v_ = 0; v_ < 8; ++v_) sh_f[{red_o} + wave * {nE} + cl_ * 8 + v_] = ov_[v_];')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}if (tid < {nE}) {{')
        o.append(f'{I}  float a_ = sh_f[{red_o} + tid];')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int w_ = 1; w_ < {NW}; ++w_) a_ += sh_f[{red_o} + w_ * {nE} + tid];')
        fenv = dict(lenv)
        fenv[at['E4']] = ('tid', 'int')
        fenv['__acc'] = ('a_', 'float')
        pre = []
        ov, ot = self.expr(c4.epi, fenv, pre, I + '  ')
        o += pre
        po = red_o + NW * nE                       # the point's output, when the projection reads it
        if pj is None:
            o.append(f'{I}  {self.store(t4[1], [fenv[a][0] for a in t4[2]], ov, ot)}')
        else:
            self.stage_floats = max(self.stage_floats, self.stage_top + NW * nE + nE)
            o.append(f'{I}  sh_f[{po} + tid] = {self.as_float(ov, ot)};')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        if pj is not None:
            self.gen_proj_tail(pj, lenv, lead, po, wp, NQP, NW, PPW, LPE, o, I)
        o.append(f'{ind}}}' + ('}' if once else ''))
        self.note(reads, writes)
        self.mark(out, ind, f'attention {t1[1]}..{t4[1]}')

    def gen_proj_tail(self, pj, lenv, lead, po, wp, NQP, NW, PPW, LPE, o, I):
        """Each lane group (LPE lanes, 8 outputs each) dots the point's output
        with one weight row; the group's first lane adds the sum into z1."""
        so, sz = pj['so'], pj['sz']
        z1, c5 = sz[1], pj['c']
        DPR, D = pj['DPR'], pj['D']
        o.append(f'{I}{{  // {so[1]}: rows [rp_ * {DPR}, +{DPR}) of {pj["st"].src}, added into {z1}')
        J = I + '  '
        o.append(f'{J}float ol_[8];')
        o.append(f'{J}{self.lds_vec_load(8, f"(sh_f + {po} + cl_ * 8)", "ol_")}')
        zenv = {a: lenv[lead[k]] for a, k in pj['pmap'].items()}
        zenv[c5.contig] = ('d_', 'int')
        za = self.addr([zenv[a][0] for a in sz[2]], self.strides(self.axes_of[z1]))
        for q in range(NQP):
            o.append(f'{J}{{ const int dl_ = {q * NW * PPW} + wave * {PPW} + sub_, d_ = rp_ * {DPR} + dl_;')
            o.append(f'{J}  float wf_[8];')
            o.append(f'{J}  unpack8({wp}[{q}], wf_);')
            o.append(f'{J}  float a_ = 0.0f;')
            o.append(f'{J}  #pragma unroll')
            o.append(f'{J}  for (int v_ = 0; v_ < 8; ++v_) a_ = fmaf(ol_[v_], wf_[v_], a_);')
            o.append(f'{J}  a_ = group_red_sum(a_, {LPE});')
            o.append(f'{J}  if (wave < {NW} && cl_ == 0 && dl_ < {DPR} && d_ < {D}) '
                     f'fxadd(S, {self.gadd(z1)} + 2u * (unsigned)({za}), a_);')
            o.append(f'{J}}}')
        o.append(f'{I}}}')
        self.mark(o, I, 'attention: projection')

    def _softmax_form(self, at):
        """Are the statistics the max-subtracted softmax, F = exp(sc - mx) and
        the weight A4 = F / hs (what the running form computes)?"""
        t1, t2, t3, _ = at['t']
        same = [('name', a) for a in at['lead'] + [at['S']]]
        at_lead = [('name', a) for a in at['lead']]
        F = ('call', 'exp', ('bin', '-', ('idx', t1[1], same), ('idx', t2[1], at_lead)))
        return t3[3][3] == F and at['c4'].A == ('bin', '/', F, ('idx', t3[1], at_lead))

    def attn_online(self, at, o, I, lenv, NPS, NPF, PPP, PPW, LPE, NW, T, nE, kq, vq, slot_env, load_kv,
                    red_o, pj, po_ref, CH, load_kv_at):
        """Scores, softmax and weighted values over chunks of CH slots:
        each lane group keeps its positions' running maximum m, sum l of
        exp(score - m) and weighted values (rescaled by exp(m_old - m_new) when
        m grows); the groups of a wave, then the waves, are combined the same
        way, and the values divided by the sum. The rows of chunk c + 1 are
        loaded while chunk c is used. The query chunk qv_ is loaded already.
        Writes the output to LDS (projection) or stores it; po_ref gets the
        LDS offset."""
        t1, t2, t3, t4 = at['t']
        c1, c4 = at['c1'], at['c4']
        NCH = -(-NPS // CH)
        o.append(f'{I}float m_ = -INFINITY, l_ = 0.0f, ov_[8];')
        o.append(f'{I}#pragma unroll')
        o.append(f'{I}for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = 0.0f;')
        first = [k for k in range(min(NPS, CH)) if k >= NPF]
        if first:
            # the first chunk's slots not loaded at the barrier
            for k in first:
                o += [I + x for x in load_kv(k, lenv, False)]
        if NCH >= ATTN_CHUNK_LOOP:
            self.attn_chunk_loop(at, o, I, lenv, PPP, PPW, LPE, NW, T, kq, vq, slot_env, CH, NCH, load_kv_at)
        for c in (range(NCH) if NCH < ATTN_CHUNK_LOOP else ()):
            ks = list(range(c * CH, min(NPS, (c + 1) * CH)))
            nxt = [k for k in range((c + 1) * CH, min(NPS, (c + 2) * CH)) if k >= NPF]
            if nxt:
                o.append(f'{I}if ({(c + 1) * CH * PPP} < {T}) {{  // rows of chunk {c + 1}')
                for k in nxt:
                    o += [I + '  ' + x for x in load_kv(k, lenv, False)]
                o.append(f'{I}}}')
            o.append(f'{I}if ({c * CH * PPP} < {T}) {{  // chunk {c}')
            J = I + '  '
            for k in ks:
                o.append(f'{J}float sk{k}_;')
                o.append(f'{J}{{ const int s{k}_ = {k * PPP} + wave * {PPW} + sub_;')
                o.append(f'{J}  float wf_[8];')
                o.append(f'{J}  unpack8({kq}[{k}], wf_);')
                o.append(f'{J}  float d_ = 0.0f;')
                o.append(f'{J}  #pragma unroll')
                o.append(f'{J}  for (int v_ = 0; v_ < 8; ++v_) d_ = fmaf(qv_[v_], wf_[v_], d_);')
                o.append(f'{J}  d_ = group_red_sum(d_, {LPE});')
                venv = dict(slot_env(k, lenv))
                venv['__acc'] = ('d_', 'float')
                pre = []
                sv, st_ = self.expr(c1.epi, venv, pre, J + '  ')
                o += pre
                o.append(f'{J}  sk{k}_ = (wave < {NW} && s{k}_ < {T}) ? {self.as_float(sv, st_)} : -INFINITY;')
                o.append(f'{J}}}')
            o.append(f'{J}float mn_ = m_;')
            for k in ks:
                o.append(f'{J}mn_ = fmaxf(mn_, sk{k}_);')
            o.append(f'{J}if (mn_ > -INFINITY) {{')
            o.append(f'{J}  const float f_ = expf(m_ - mn_);')
            o.append(f'{J}  l_ *= f_;')
            o.append(f'{J}  #pragma unroll')
            o.append(f'{J}  for (int v_ = 0; v_ < 8; ++v_) ov_[v_] *= f_;')
            for k in ks:
                o.append(f'{J}  {{ const float p_ = sk{k}_ > -INFINITY ? expf(sk{k}_ - mn_) : 0.0f;')
                o.append(f'{J}    l_ += p_;')
                o.append(f'{J}    float wf_[8];')
                o.append(f'{J}    unpack8({vq}[{k}], wf_);')
                o.append(f'{J}    #pragma unroll')
                o.append(f'{J}    for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = fmaf(p_, wf_[v_], ov_[v_]);')
                o.append(f'{J}  }}')
            o.append(f'{J}  m_ = mn_;')
            o.append(f'{J}}}')
            o.append(f'{I}}}')
        self.mark(o, I, 'attention: chunks')
        # the wave's lane groups, then the waves
        o.append(f'{I}{{ const float M_ = wave_red_max_hi(m_, {LPE});')
        o.append(f'{I}  const float f_ = m_ > -INFINITY ? expf(m_ - M_) : 0.0f;')
        o.append(f'{I}  const float L_ = wave_red_sum_hi(l_ * f_, {LPE});')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = wave_red_sum_hi(ov_[v_] * f_, {LPE});')
        red_m = red_o + NW * nE
        po = red_m + 2 * 8
        self.stage_floats = max(self.stage_floats, self.stage_top + NW * nE + 16 + nE)
        o.append(f'{I}  if (wave < {NW} && sub_ == 0) {{')
        o.append(f'{I}    #pragma unroll')
        o.append(f'{I}    for (int v_ = 0; v_ < 8; ++v_) sh_f[{red_o} + wave * {nE} + cl_ * 8 + v_] = ov_[v_];')
        o.append(f'{I}    if (lane == 0) {{ sh_f[{red_m} + wave] = M_; sh_f[{red_m + 8} + wave] = L_; }}')
        o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}if (tid < {nE}) {{')
        o.append(f'{I}  float M_ = sh_f[{red_m}];')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int w_ = 1; w_ < {NW}; ++w_) M_ = fmaxf(M_, sh_f[{red_m} + w_]);')
        o.append(f'{I}  float L_ = 0.0f, a_ = 0.0f;')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int w_ = 0; w_ < {NW}; ++w_) {{')
        o.append(f'{I}    const float mw_ = sh_f[{red_m} + w_];')
        o.append(f'{I}    const float f_ = mw_ > -INFINITY ? expf(mw_ - M_) : 0.0f;')
        o.append(f'{I}    L_ = fmaf(sh_f[{red_m + 8} + w_], f_, L_);')
        o.append(f'{I}    a_ = fmaf(sh_f[{red_o} + w_ * {nE} + tid], f_, a_);')
        o.append(f'{I}  }}')
        o.append(f'{I}  a_ = a_ / L_;')
        fenv = dict(lenv)
        fenv[at['E4']] = ('tid', 'int')
        fenv['__acc'] = ('a_', 'float')
        pre = []
        ov, ot = self.expr(c4.epi, fenv, pre, I + '  ')
        o += pre
        if pj is None:
            o.append(f'{I}  {self.store(t4[1], [fenv[a][0] for a in t4[2]], ov, ot)}')
        else:
            o.append(f'{I}  sh_f[{po} + tid] = {self.as_float(ov, ot)};')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        self.mark(o, I, 'attention: combine')
        po_ref.append(po)

    def attn_chunk_loop(self, at, o, I, lenv, PPP, PPW, LPE, NW, T, kq, vq, slot_env, CH, NCH, load_kv_at):
        """The chunks of ``attn_online`` as a run-time loop: the current
        chunk's rows in kc_/vc_ (the first chunk's from kq/vq), the next
        chunk's loaded into kn_/vn_ (``load_kv_at``: the rows of a slot given
        as a C expression) while the current one is used. The operations and
        their order are those of the unrolled chunks."""
        c1 = at['c1']
        o.append(f'{I}vh_u32x4 kc_[{CH}], vc_[{CH}], kn_[{CH}], vn_[{CH}];')
        for j in range(CH):
            o.append(f'{I}kc_[{j}] = {kq}[{j}]; vc_[{j}] = {vq}[{j}];')
        o.append(f'{I}for (int c_ = 0; c_ < {NCH}; ++c_) {{')
        J0 = I + '  '
        o.append(f'{J0}if ((c_ + 1) * {CH * PPP} < {T}) {{  // rows of the next chunk')
        for j in range(CH):
            o += [J0 + '  ' + x for x in load_kv_at(f'n{j}', f'(c_ + 1) * {CH} + {j}', lenv,
                                                          f'kn_[{j}]', f'vn_[{j}]')]
        o.append(f'{J0}}}')
        o.append(f'{J0}if (c_ * {CH * PPP} < {T}) {{  // this chunk')
        J = J0 + '  '
        for j in range(CH):
            k = f'c{j}'
            o.append(f'{J}float sk{j}_;')
            o.append(f'{J}{{ const int s{k}_ = (c_ * {CH} + {j}) * {PPP} + wave * {PPW} + sub_;')
            o.append(f'{J}  float wf_[8];')
            o.append(f'{J}  unpack8(kc_[{j}], wf_);')
            o.append(f'{J}  float d_ = 0.0f;')
            o.append(f'{J}  #pragma unroll')
            o.append(f'{J}  for (int v_ = 0; v_ < 8; ++v_) d_ = fmaf(qv_[v_], wf_[v_], d_);')
            o.append(f'{J}  d_ = group_red_sum(d_, {LPE});')
            venv = dict(slot_env(k, lenv))
            venv['__acc'] = ('d_', 'float')
            pre = []
            sv, st_ = self.expr(c1.epi, venv, pre, J + '  ')
            o += pre
            o.append(f'{J}  sk{j}_ = (wave < {NW} && s{k}_ < {T}) ? {self.as_float(sv, st_)} : -INFINITY;')
            o.append(f'{J}}}')
        o.append(f'{J}float mn_ = m_;')
        for j in range(CH):
            o.append(f'{J}mn_ = fmaxf(mn_, sk{j}_);')
        o.append(f'{J}if (mn_ > -INFINITY) {{')
        o.append(f'{J}  const float f_ = expf(m_ - mn_);')
        o.append(f'{J}  l_ *= f_;')
        o.append(f'{J}  #pragma unroll')
        o.append(f'{J}  for (int v_ = 0; v_ < 8; ++v_) ov_[v_] *= f_;')
        for j in range(CH):
            o.append(f'{J}  {{ const float p_ = sk{j}_ > -INFINITY ? expf(sk{j}_ - mn_) : 0.0f;')
            o.append(f'{J}    l_ += p_;')
            o.append(f'{J}    float wf_[8];')
            o.append(f'{J}    unpack8(vc_[{j}], wf_);')
            o.append(f'{J}    #pragma unroll')
            o.append(f'{J}    for (int v_ = 0; v_ < 8; ++v_) ov_[v_] = fmaf(p_, wf_[v_], ov_[v_]);')
            o.append(f'{J}  }}')
        o.append(f'{J}  m_ = mn_;')
        o.append(f'{J}}}')
        o.append(f'{J0}}}')
        for j in range(CH):
            o.append(f'{J0}kc_[{j}] = kn_[{j}]; vc_[{j}] = vn_[{j}];')
        o.append(f'{I}}}')

    def _subst(self, e, repl):
        """e with reads of the named group values replaced by C variables:
        (expression, the environment entries binding them)."""
        def f(n):
            if n[0] == 'idx' and n[1] in repl:
                return ('name', '__v_' + n[1])
            return n
        return self.rebuild_expr(e, f), {('__v_' + k): (v, 'float') for k, v in repl.items()}
