"""Streamed contractions with several rows on the matrix cores.

A stream ``y[r.., p] = EPI(fold sum k: A[r.., k] * W[p, k])`` with 4 to 64
rows r (the batch) and fp16 weights runs on ``v_mfma_f32_16x16x32_f16``:
rows are the MFMA's M (padded to 16 with zeros; beyond 16 rows, one tile per
16 rows, each with its own accumulators), a tile of 16 consecutive
output points its N, and the fold its K, 32 at a time. Lane l of a wave holds
A[l % 16][k0 + 8 (l / 16) ..+8], W[k0 + 8 (l / 16) ..+8][point l % 16] (one
16-byte load from the point's row of the weight copy) and, after the loop,
y[4 (l / 16) + v][point l % 16] for v < 4.

The other factor is fp32; it is split into fp16 halves a = hi + lo (hi the
nearest fp16, lo the nearest fp16 to the exact remainder), so a keeps 22
significant bits (the weights are fp16 already, and every product is exact).
Values beyond the fp16 range (65504) are not representable on this path.
With at most 8 rows both halves share one MFMA: rows 0-7 of the A tile hold
the rows' hi halves and rows 8-15 their lo halves, the remainder scaled by
2^11 (exact) so it keeps 11 bits at any magnitude; the result rows r and
r + 8 (lanes l and l + 32) are combined as hi + lo / 2048 after the loop.
With more rows hi and lo go through separate MFMAs into one accumulator.

Work split: a block's points form NT tiles. With at least as many tiles as
compute waves, wave w makes tiles w, w + NW, .. over the whole fold; with
fewer, KW waves share a tile, each over its own range of the fold, and the
partial tiles are added through LDS in wave order (a fixed order, so results
do not depend on timing). The weights of a wave's share are loaded at the
barrier before the site when they fit in the prefetch register budget, else
streamed through two register sets of ``mfma_pipe`` k-blocks each. Every
weight fragment a wave loads meets all of its row tiles.

The halves of the other factor live in LDS. When those of all rows over the
whole fold would exceed ``MFMA_HALVES_MAX`` bytes (beyond 16 rows only), the
fold goes through LDS in chunks of whole k-blocks, every wave taking the
same part of each chunk, and the weights are streamed.
"""
from __future__ import annotations

from .analysis import LowerError, top_folds

MFMA_ROWS_MIN = 4            # rows from which a stream runs on the matrix cores
MFMA_PIPES = (2, 1)          # k-blocks of weights per register set when not prefetched (two sets: the
                             # next set's loads are in flight while one is used), tried in turn at each
                             # prefetch budget; GPT-2 small B=8, same box, alternating order: 321 us per
                             # step at 2, 324.6 at 1, equal tokens and logits; 3 spills 57 registers at
                             # the full budget
MFMA_POINTS_MIN = 8          # points a block must make (of a tile's 16 columns)
MFMA_ROWS_MAX = 64           # rows a stream may take: beyond 16, in 16-row tiles (each a tile of its own)
MFMA_HALVES_MAX = 100 * 1024  # bytes of LDS the fp16 halves of the other factor take at most beyond 16 rows
                             # (the fold then goes through LDS in chunks of whole 32-deep k-blocks)
SPLIT_ADD_BYTES = 32         # beyond 16 rows, the cost of one fixed-point add of a fold split in bytes read
SPLIT_TILES = 4              # column tiles a fold split's point group takes at most, up to 16 rows (16 beyond)
SPLIT_TILES_PACKED = 2       # the same at 8 rows or fewer: GPT-2 medium at 8 rows 848.8 -> 741.9 us per
                             # step (3 tiles 744.7, 1 tile 872.0), small at 8 rows 293.9 -> 290.6, at 4
                             # and 6 rows 1% better; at 10 rows 2 tiles lose (382.8 -> 391.7)


class MfmaMixin:
    def mfma_ok(self, c, st, points=True):
        """Can stream st (of contraction c) run on the matrix cores, with at
        least half of a tile's 16 columns holding points of the block (unless
        ``points`` is off: a fold split over blocks sets its own points)?"""
        R = self.size(c.reg_axes)
        PPB = -(-self.size(st.pts) // self.grid)
        if not (self.res[st.src][1] == 'f16' and MFMA_ROWS_MIN <= R <= MFMA_ROWS_MAX and st.K % 32 == 0
                and st.c0 % 8 == 0 and st.rowlen % 8 == 0 and (PPB >= MFMA_POINTS_MIN or not points)):
            return False
        # beyond one row tile the other factor is split into halves chunk by
        # chunk from where it lives: a value laid out [rows, fold], read at
        # exactly those axes (``mfma_reachable`` confirms where it is stored)
        if R <= 16:
            return True
        A, want = c.A, list(c.reg_axes) + list(c.fold_axes)
        return (A[0] == 'idx' and A[1] in self.axes_of and list(self.axes_of[self.root(A[1])]) == want
                and list(A[2]) == [('name', a) for a in want])

    def mfma_reachable(self, c, st):
        """At code generation: a stream of more than 16 rows reads its other
        factor in place, from LDS (private) or as plain fp32 global scratch."""
        return (self.size(c.reg_axes) <= 16 or self.direct_lds(c, c.reg_axes) is not None
                or self.mfma_global_src(c, c.reg_axes, st.K) is not None)

    @staticmethod
    def mfma_rows(R, nkb):
        """(row tiles, k-blocks per fold chunk, fold chunks) of a stream of R
        rows over nkb k-blocks: up to 16 rows one tile and the whole fold;
        beyond, 16-row tiles and, when the halves of all rows over the whole
        fold exceed MFMA_HALVES_MAX bytes, chunks of the fold that fit."""
        if R <= 16:
            return 1, nkb, 1
        RT = -(-R // 16)
        if 2 * R * (nkb * 64 + 16) <= MFMA_HALVES_MAX:
            return RT, nkb, 1
        cb = max(1, (MFMA_HALVES_MAX // (2 * R) - 16) // 64)
        return RT, cb, -(-nkb // cb)

    def gen_stream_mfma(self, s, c, st, fused, out, ind):
        name = s[1]
        reads, writes = self.site_io(s, c, fused)
        self.sync(reads, writes, out, ind, name)
        self.plan.append((self.show_stmt(s), 'stream' + (' (transposed copy)' if st.pack else '') + ' mfma'
                          + (f' +{len(fused)} fused' if fused else '')))
        for _, t, _ in fused:
            self.plan.append((self.show_stmt(t), f'epilogue of {name}'))
        K, NKB = st.K, st.K // 32
        NW = self.NWAVE - 1
        P = self.size(st.pts)
        PPB = -(-P // self.grid)
        reg = c.reg_axes
        R = self.size(reg)
        NT = -(-PPB // 16)
        RT, CB, NC = self.mfma_rows(R, NKB)   # row tiles (each tile's accumulators); k-blocks per fold chunk, chunks
        if NT >= NW:
            TPW, KW = -(-NT // NW), 1
        else:
            TPW, KW = 1, NW // NT
        KBW = -(-CB // KW)
        prefetch = NC == 1 and TPW * KBW * 4 <= self.pf_budget
        sid = self.fresh('m')
        CT = NW * 64                          # the epilogue: one (row, point) item per compute thread
        NI = -(-(R * PPB) // CT)
        geo = dict(P=P, PPB=PPB, NW=NW, NT=NT, TPW=TPW, KW=KW, NKB=CB, KBW=KBW, R=R, reg=list(reg), CT=CT)
        rr = self.rsrc(st.src)
        rs = self.res_strides(st.src)
        w16 = self.w16('stream')
        I = ind + '  '
        o = out

        def wload(i, kb, dst, cond='true'):
            """Lines loading the weight fragment of slot i, k-block kb (C
            expressions) into dst (zeros where there is no point)."""
            lines = [f'{{ const int n_ = ({self.mfma_tile(geo, i)}) * 16 + (lane & 15);',
                     '  const int p_ = (int)blockIdx.x * %d + n_;' % PPB,
                     f'  if (mok_ && ({cond}) && ({self.mfma_tile(geo, i)}) < {NT} && n_ < {PPB} && p_ < {P}) {{']
            env = self.decode('p_', st.pts, lines, '    ', prefix='sp_')
            pre = []
            ix = [self.index(x, env, pre, '    ') for x in st.prefix_idx]
            lines += pre
            base = self.addr(ix, rs[:-1]) if ix else '0'
            lines.append(f'    {dst} = {w16}({rr}, (unsigned)({base}) + {st.c0}u + (unsigned)(({kb}) * 32 + (lane >> 4) * 8));')
            lines.append(f'  }} else {dst} = vh_u32x4{{0u, 0u, 0u, 0u}};')
            lines.append('}')
            return lines

        wm = f'wm_{sid}'
        if prefetch:
            self.decls.append(f'vh_u32x4 {wm}[{TPW}][{KBW}];')
            unsafe = self.unsafe_early()
            caps = {}

            def make(step_override):
                saved = self.override_step(step_override)
                try:
                    lines = [f'if (wave < {NW}) {{'] + ['  ' + x for x in self.mfma_role(geo)]
                    for i in range(TPW):
                        for j in range(KBW):
                            lines += ['  ' + x for x in wload(i, f'mk0_ + {j}', f'{wm}[{i}][{j}]', f'mk0_ + {j} < mk1_')]
                    for q in range(NI):
                        pre = f'pf_{sid}_{q}_'
                        self.capture = {'prefix': pre, 'loads': [], 'unsafe': unsafe}
                        try:
                            self.epilogue(s, c, fused, self.mfma_env(st, geo), '0.0f', [], '')
                            loads = self.capture['loads']
                        finally:
                            self.capture = None
                        caps[pre] = [(n, k) for n, _, k in loads]
                        if loads:
                            lines += ['  ' + x for x in self.mfma_item(st, geo, q, [f'{n} = {t};' for n, t, _ in loads])]
                    return lines + ['}']
                finally:
                    self.restore_step(saved)
            self.place_prefetch(make, o, ind)
            for regs in caps.values():
                for n, k in regs:
                    self.decls.append(f'{self.cap_ctype(k)} {n};')
        o.append(f'{ind}{{  // stream {name} on the matrix cores: {P} points x {K} from {st.src}, rows={R}, '
                 f'points/block={PPB}, tiles={NT}, tiles/wave={TPW}, waves/tile={KW}'
                 + (f', {RT} row tiles, fold in {NC} chunks of {CB} k-blocks' if RT > 1 else '')
                 + (' prefetched' if prefetch else ''))
        o += [I + x for x in self.mfma_role(geo)]
        self.stream_part[self.root(name)] = dict(pts=list(st.pts), PPB=PPB, P=P, reg=list(reg))
        # LDS: [fp32 copy of the other factor, if it has to be made] [hi] [lo] [partial tiles] [values]
        top = self.lds_floats + self.stage_top
        direct = self.direct_lds(c, reg)
        src = None
        if direct is None:
            src = self.mfma_global_src(c, reg, K)
            if src is None:
                self.stage_A(c, reg, 0, R, R, K, str(top), o, I)
                direct, top = str(top), top + R * K
        SAB = CB * 64 + 16                    # bytes per row of a half array (padded against bank conflicts)
        packed = R <= 8                       # hi rows 0-7 and lo rows 8-15 of one A tile
        ah = top * 4
        al = ah + (8 if packed else R) * SAB
        top = (al + R * SAB) // 4
        red = top
        if KW > 1:
            top += NW * 64 * 4 * RT
        accb = top                            # the sums, [row][own point]
        top += -(-R * PPB // 4) * 4
        if NC == 1:
            self.mfma_split(direct, src, R, K, SAB, ah, al, o, I, scaled=packed)
            self.mark(o, I, f'stream {name}: halves')
        # values of the site (as in the other streams)
        fused_ids = {id(t) for _, t, _ in fused}
        made = [s] + [t for kind, t, _ in fused if kind == 'let']
        self.skip_store = {t[1] for t in made if self.epi_only(t[1], fused_ids)}
        self.out_stage = {}
        for t in made:
            n = t[1]
            if n in self.skip_store or not self.stage_out_ok(t, reg, st.pts, R, PPB):
                continue
            self.out_stage[n] = (top, PPB, list(reg), list(st.pts))
            top += -(-R * PPB // 4) * 4
        self.stage_floats = max(self.stage_floats, top - self.lds_floats)
        # the products
        if RT == 1:
            o.append(f'{I}vh_f32x4 acc_[{TPW}];')
            o.append(f'{I}#pragma unroll')
            o.append(f'{I}for (int i_ = 0; i_ < {TPW}; ++i_) acc_[i_] = vh_f32x4{{0.f, 0.f, 0.f, 0.f}};')
        else:
            self.mfma_acc_rows(TPW, RT, o, I)

        def kstep(kb, wsrc, J):
            """Lines of one k-block (C expression kb, relative to mk0_) from weight registers wsrc(i)."""
            if packed:
                return self.mfma_kstep_packed(f'mk0_ + {kb}', wsrc, TPW, R, SAB, ah, J)
            if RT == 1:
                lines = [f'{J}{{ const int kb_ = mk0_ + {kb};',
                         f'{J}  const int ar_ = lane & 15, ak_ = kb_ * 32 + (lane >> 4) * 8;',
                         f'{J}  const vh_u32x4 ah_ = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {ah} + ar_ * {SAB} + ak_ * 2) '
                         f': vh_u32x4{{0u, 0u, 0u, 0u}};',
                         f'{J}  const vh_u32x4 al_ = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {al} + ar_ * {SAB} + ak_ * 2) '
                         f': vh_u32x4{{0u, 0u, 0u, 0u}};']
                for i in range(TPW):
                    lines.append(f'{J}  acc_[{i}] = vh_mfma(ah_, {wsrc(i)}, acc_[{i}]);')
                    lines.append(f'{J}  acc_[{i}] = vh_mfma(al_, {wsrc(i)}, acc_[{i}]);')
                lines.append(f'{J}}}')
                return lines
            # row tiles: every weight fragment multiplies each 16-row tile; the
            # halves in LDS hold the current fold chunk (columns from ck0_)
            return self.mfma_kstep_rows(f'mk0_ + {kb}', ' - ck0_' if NC > 1 else '', wsrc, TPW, RT, R, SAB,
                                        ah, al, J)

        def streamed(J):
            """The wave's k-blocks [mk0_, mk1_) with weights streamed through two register sets."""
            D = self.mfma_pipe
            o.append(f'{J}vh_u32x4 wb0_[{TPW}][{D}], wb1_[{TPW}][{D}];')
            for i in range(TPW):
                for d in range(D):
                    o.extend(J + x for x in wload(i, f'mk0_ + {d}', f'wb0_[{i}][{d}]', f'mk0_ + {d} < mk1_'))
            o.append(f'{J}for (int c0_ = 0; c0_ < {KBW}; c0_ += {2 * D}) {{')
            J2 = J + '  '
            for half, (cur, nxt) in enumerate((('wb0_', 'wb1_'), ('wb1_', 'wb0_'))):
                ahead = f'c0_ + {(half + 1) * D}'
                for i in range(TPW):
                    for d in range(D):
                        o.extend(J2 + x for x in wload(i, f'mk0_ + {ahead} + {d}', f'{nxt}[{i}][{d}]',
                                                       f'mk0_ + {ahead} + {d} < mk1_'))
                for d in range(D):
                    kb = f'c0_ + {half * D + d}'
                    o.append(f'{J2}if (mk0_ + {kb} < mk1_)')
                    o.extend(kstep(kb, lambda i, cur=cur, d=d: f'{cur}[{i}][{d}]', J2 + '  '))
            o.append(f'{J}}}')

        if NC == 1:
            o.append(f'{I}if (mok_) {{')
            J = I + '  '
            if prefetch:
                for j in range(KBW):
                    o.append(f'{J}if (mk0_ + {j} < mk1_)')
                    o += kstep(str(j), lambda i, j=j: f'{wm}[{i}][{j}]', J + '  ')
            else:
                streamed(J)
            o.append(f'{I}}}')
        else:
            # the fold in chunks: each chunk's halves into LDS, then every wave
            # takes its part of the chunk's k-blocks (parts in the same order
            # in every chunk, so each wave's sum covers the same part of each)
            o.append(f'{I}for (int ch_ = 0; ch_ < {NC}; ++ch_) {{')
            J0 = I + '  '
            o.append(f'{J0}const int ck0_ = ch_ * {CB}, ckn_ = min({CB}, {NKB} - ck0_);')
            self.mfma_split_chunk(direct, src, R, K, SAB, ah, al, o, J0)
            o.append(f'{J0}if (mok_) {{')
            J = J0 + '  '
            o.append(f'{J}const int mk0_ = ck0_ + mkp_ * ckn_ / {KW}, mk1_ = ck0_ + (mkp_ + 1) * ckn_ / {KW};')
            streamed(J)
            o.append(f'{J0}}}')
            o.append(f'{I}}}')
        self.mark(o, I, f'stream {name}: products')
        if KW > 1 and RT > 1:
            self.mfma_parts_rows(KW, NT, RT, red, o, I)
        elif KW > 1:
            # partial tiles of the later parts of the fold, added in part order
            o.append(f'{I}if (mok_ && mkp_ > 0) *(vh_f32x4*)(sh_f + {red} + (wave * 64 + lane) * 4) = acc_[0];')
            o.append(f'{I}vh_lds_sync();')
            o.append(f'{I}if (mok_ && mkp_ == 0) {{')
            for q in range(1, KW):
                o.append(f'{I}  acc_[0] += *(const vh_f32x4*)(sh_f + {red} + ((wave + {q * NT}) * 64 + lane) * 4);')
            o.append(f'{I}}}')
        # the sums into LDS [row][own point] (lane l holds rows 4 (l / 16) ..+4 of
        # point l % 16 of each of its tiles); then every compute thread finishes
        # one (row, point) item at a time, consecutive threads consecutive points
        o.append(f'{I}if (mok_ && mkp_ == 0) {{')
        if packed:
            o += self.mfma_combine_packed(TPW, I + '  ')
        for i in range(TPW):
            o.append(f'{I}  {{ const int n_ = ({self.mfma_tile(geo, i)}) * 16 + (lane & 15);')
            o.append(f'{I}    if (({self.mfma_tile(geo, i)}) < {NT} && n_ < {PPB}) {{')
            o.append(f'{I}      #pragma unroll')
            o.append(f'{I}      for (int v_ = 0; v_ < 4; ++v_) {{')
            if RT == 1:
                o.append(f'{I}        const int r_ = (lane >> 4) * 4 + v_;')
                o.append(f'{I}        if (r_ < {R}) sh_f[{accb} + r_ * {PPB} + n_] = acc_[{i}][v_];')
            else:
                for rt in range(RT):
                    o.append(f'{I}        {{ const int r_ = {rt * 16} + (lane >> 4) * 4 + v_;')
                    o.append(f'{I}          if (r_ < {R}) sh_f[{accb} + r_ * {PPB} + n_] = acc_[{i}][{rt}][v_]; }}')
            o.append(f'{I}      }}')
            o.append(f'{I}    }}')
            o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        for q in range(NI):
            body = []
            if prefetch:
                self.capture = {'prefix': f'pf_{sid}_{q}_', 'loads': [], 'unsafe': unsafe}
            try:
                self.epilogue(s, c, fused, self.mfma_env(st, geo), f'sh_f[{accb} + e_]', body, '')
            finally:
                self.capture = None
            o += [I + x for x in self.mfma_item(st, geo, q, body)]
        if self.out_stage:
            self.write_out(P, PPB, R, o, I)
            self.mark(o, I, f'stream {name}: write out')
        self.stream_lds = {self.root(n): (base, PPB, R) for n, (base, _, _, _) in self.out_stage.items()}
        self.skip_store, self.out_stage = set(), {}
        o.append(f'{ind}}}')
        self.note(reads, writes)
        self.mark(out, ind, f'stream {name}')

    # ------------------------------------------------------------ pieces
    @staticmethod
    def mfma_role(geo):
        """Lines binding this wave's share: mok_ (takes part), mkp_ (its part of
        the fold), mt_ (its first tile), mk0_ / mk1_ (its k-blocks)."""
        NW, NT, KW, NKB = geo['NW'], geo['NT'], geo['KW'], geo['NKB']
        if KW == 1:
            return [f'const bool mok_ = wave < {NW} && wave < {NT};',
                    'const int mkp_ = 0, mt_ = wave, mk0_ = 0, mk1_ = %d;' % NKB]
        return [f'const bool mok_ = wave < {NT * KW};',
                f'const int mkp_ = wave / {NT}, mt_ = wave % {NT};',
                f'const int mk0_ = mkp_ * {NKB} / {KW}, mk1_ = (mkp_ + 1) * {NKB} / {KW};']

    @staticmethod
    def mfma_tile(geo, i):
        return f'mt_ + {i * geo["NW"]}' if i else 'mt_'

    def mfma_env(self, st, geo):
        env = {a: (f'ep_{a}', 'int') for a in st.pts}
        for a in geo['reg']:
            env[a] = (f'er_{a}', 'int')
        return env

    def mfma_item(self, st, geo, q, body):
        """Lines binding row r_ and point p_ of this thread's item q (item
        e_ = tid + q * CT of the block's rows x points, point fastest) around
        ``body``."""
        PPB, CT = geo['PPB'], geo['CT']
        lines = [f'{{ const int e_ = tid + {q * CT};',
                 f'  const int r_ = e_ / {PPB}, n_ = e_ - r_ * {PPB};',
                 f'  const int p_ = (int)blockIdx.x * {PPB} + n_;',
                 f'  if (tid < {CT} && e_ < {geo["R"] * PPB} && p_ < {geo["P"]}) {{']
        self.decode('p_', st.pts, lines, '    ', prefix='ep_')
        if geo['reg']:
            self.decode('r_', geo['reg'], lines, '    ', prefix='er_')
        lines += ['    ' + x for x in body]
        lines += ['  }', '}']
        return lines

    def mfma_global_src(self, c, reg, K):
        """Global scratch offset of the other factor when it is a plain fp32
        value laid out [reg axes, fold axes] (read with 16-byte loads), else None."""
        A = c.A
        if A[0] != 'idx' or A[1] not in self.axes_of:
            return None
        r = self.root(A[1])
        want = list(reg) + list(c.fold_axes)
        if (r in self.private or r in self.fx or r in self.peel_active or r not in self.g
                or list(self.axes_of[r]) != want or list(A[2]) != [('name', a) for a in want] or K % 8):
            return None
        return self.g[r]

    def mfma_kstep_packed(self, kb, wsrc, TPW, R, SAB, ah, J):
        """One k-block (C expression kb) with hi and lo halves in one A tile:
        lane l reads row l % 16 of the [16][SAB] half array (rows 8-15: lo)."""
        lines = [f'{J}{{ const int kb_ = {kb};',
                 f'{J}  const int ar_ = lane & 15, ak_ = kb_ * 32 + (lane >> 4) * 8;',
                 f'{J}  const vh_u32x4 a_ = (ar_ & 7) < {R} ? *(const vh_u32x4*)((const char*)sh_f + {ah} + ar_ * {SAB} '
                 f'+ ak_ * 2) : vh_u32x4{{0u, 0u, 0u, 0u}};']
        for i in range(TPW):
            lines.append(f'{J}  acc_[{i}] = vh_mfma(a_, {wsrc(i)}, acc_[{i}]);')
        lines.append(f'{J}}}')
        return lines

    def mfma_combine_packed(self, TPW, J):
        """Lanes l and l + 32 hold the hi and lo sums of the same rows and
        points: every lane gets hi + lo / 2048 (lanes 32-63 then hold rows 8-15,
        which the callers skip)."""
        lines = []
        for i in range(TPW):
            for v in range(4):
                lines.append(f'{J}acc_[{i}][{v}] = vh_pair32(acc_[{i}][{v}], vh_hilo);')
        return lines

    def mfma_split(self, direct, src, R, K, SAB, ah, al, o, I, scaled=False):
        """The other factor (rows x K fp32, in LDS at float offset ``direct``
        or in global scratch at ``src``) into fp16 halves in LDS; ``scaled``:
        the lo half as fp16((v - hi) * 2048)."""
        K8 = K // 8
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}for (int e_ = tid; e_ < {R * K8}; e_ += {self.BLOCK}) {{')
        o.append(f'{I}  const int r_ = e_ / {K8}, k8_ = e_ - r_ * {K8};')
        o.append(f'{I}  float v_[8];')
        if direct is not None:
            o.append(f'{I}  const float* s_ = sh_f + {direct} + r_ * {K} + k8_ * 8;')
            o.append(f'{I}  {self.lds_vec_load(8, "s_", "v_")}')
        else:
            o.append(f'{I}  const vh_f32x4 x0_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + k8_ * 8)), '
                     f'x1_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + k8_ * 8 + 4));')
            o.append(f'{I}  v_[0] = x0_.x; v_[1] = x0_.y; v_[2] = x0_.z; v_[3] = x0_.w; '
                     f'v_[4] = x1_.x; v_[5] = x1_.y; v_[6] = x1_.z; v_[7] = x1_.w;')
        o.append(f'{I}  vh_u32x4 h_, l_;')
        o.append(f'{I}  {"vh_split8s" if scaled else "vh_split8"}(v_, h_, l_);')
        o.append(f'{I}  if (vh_beyond_half8(v_)) stc_u(bar + VH_BAR_ERROR, VH_ERR_RANGE);')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {ah} + r_ * {SAB} + k8_ * 16) = h_;')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {al} + r_ * {SAB} + k8_ * 16) = l_;')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')

    @staticmethod
    def mfma_acc_rows(TPW, RT, o, I):
        """Accumulators of TPW column tiles x RT row tiles."""
        o.append(f'{I}vh_f32x4 acc_[{TPW}][{RT}];')
        o.append(f'{I}#pragma unroll')
        o.append(f'{I}for (int i_ = 0; i_ < {TPW}; ++i_)')
        o.append(f'{I}  #pragma unroll')
        o.append(f'{I}  for (int r_ = 0; r_ < {RT}; ++r_) acc_[i_][r_] = vh_f32x4{{0.f, 0.f, 0.f, 0.f}};')

    @staticmethod
    def mfma_kstep_rows(kb, rel, wsrc, TPW, RT, R, SAB, ah, al, J):
        """One k-block (C expression kb; its LDS column ``kb{rel}``) of TPW
        column tiles over RT row tiles: lane l reads rows rt * 16 + l % 16 of
        the hi and lo arrays, and each weight fragment meets every row tile."""
        lines = [f'{J}{{ const int kb_ = {kb};',
                 f'{J}  const int ak_ = (kb_{rel}) * 32 + (lane >> 4) * 8;',
                 f'{J}  vh_u32x4 ah_[{RT}], al_[{RT}];',
                 f'{J}  #pragma unroll',
                 f'{J}  for (int rt_ = 0; rt_ < {RT}; ++rt_) {{',
                 f'{J}    const int ar_ = rt_ * 16 + (lane & 15);',
                 f'{J}    ah_[rt_] = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {ah} + ar_ * {SAB} + ak_ * 2) '
                 f': vh_u32x4{{0u, 0u, 0u, 0u}};',
                 f'{J}    al_[rt_] = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {al} + ar_ * {SAB} + ak_ * 2) '
                 f': vh_u32x4{{0u, 0u, 0u, 0u}};',
                 f'{J}  }}']
        for i in range(TPW):
            lines += [f'{J}  #pragma unroll',
                      f'{J}  for (int rt_ = 0; rt_ < {RT}; ++rt_) {{',
                      f'{J}    acc_[{i}][rt_] = vh_mfma(ah_[rt_], {wsrc(i)}, acc_[{i}][rt_]);',
                      f'{J}    acc_[{i}][rt_] = vh_mfma(al_[rt_], {wsrc(i)}, acc_[{i}][rt_]);',
                      f'{J}  }}']
        lines.append(f'{J}}}')
        return lines

    @staticmethod
    def mfma_parts_rows(KW, NT, RT, red, o, I):
        """Partial tiles (all row tiles) of the later parts of the fold added
        to the first part's, in part order, through LDS (one tile per wave)."""
        o.append(f'{I}if (mok_ && mkp_ > 0) {{')
        for rt in range(RT):
            o.append(f'{I}  *(vh_f32x4*)(sh_f + {red} + ((wave * {RT} + {rt}) * 64 + lane) * 4) = acc_[0][{rt}];')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}if (mok_ && mkp_ == 0) {{')
        for q in range(1, KW):
            for rt in range(RT):
                o.append(f'{I}  acc_[0][{rt}] += *(const vh_f32x4*)(sh_f + {red} + (((wave + {q * NT}) * {RT} + {rt}) * 64 '
                         f'+ lane) * 4);')
        o.append(f'{I}}}')

    def mfma_split_chunk(self, direct, src, R, K, SAB, ah, al, o, I):
        """The fold chunk of k-blocks [ck0_, ck0_ + ckn_) (C variables) of the
        other factor (R rows x K fp32, in LDS at float offset ``direct`` or in
        global scratch at ``src``) into fp16 hi and lo halves in LDS, chunk
        column 0 first."""
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}for (int e_ = tid; e_ < {R} * ckn_ * 4; e_ += {self.BLOCK}) {{')
        o.append(f'{I}  const int r_ = e_ / (ckn_ * 4), k8_ = e_ - r_ * (ckn_ * 4);')
        o.append(f'{I}  const int col_ = ck0_ * 32 + k8_ * 8;')
        o.append(f'{I}  float v_[8];')
        if direct is not None:
            o.append(f'{I}  const float* s_ = sh_f + {direct} + r_ * {K} + col_;')
            o.append(f'{I}  {self.lds_vec_load(8, "s_", "v_")}')
        else:
            o.append(f'{I}  const vh_f32x4 x0_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + col_)), '
                     f'x1_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + col_ + 4));')
            o.append(f'{I}  v_[0] = x0_.x; v_[1] = x0_.y; v_[2] = x0_.z; v_[3] = x0_.w; '
                     f'v_[4] = x1_.x; v_[5] = x1_.y; v_[6] = x1_.z; v_[7] = x1_.w;')
        o.append(f'{I}  vh_u32x4 h_, l_;')
        o.append(f'{I}  vh_split8(v_, h_, l_);')
        o.append(f'{I}  if (vh_beyond_half8(v_)) stc_u(bar + VH_BAR_ERROR, VH_ERR_RANGE);')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {ah} + r_ * {SAB} + k8_ * 16) = h_;')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {al} + r_ * {SAB} + k8_ * 16) = l_;')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')

    # ------------------------------------------------------------ fold split over blocks
    def split_of(self, s):
        """A multi-row stream with too few points per block for a matrix tile
        whose statement adds the sum to a base, y = BASE + fold sum k: A * W:
        the fold is split over blocks too, each block multiplying a slice of A
        into tiles of its point group, and the partial tiles are added into y
        kept as a 64-bit fixed-point sum (exact: the order of the adds does not
        change it), whose BASE is stored in the phase before. Returns the
        geometry, or None."""
        if s[0] != 'let' or self.place.get(id(s)) not in ('tile', 'lane'):
            return None
        c = self.info[id(s)]
        st = self.stream_of(c)
        if st is None:
            return None
        name, r = s[1], self.root(s[1])
        R = self.size(c.reg_axes)
        P = self.size(st.pts)
        if not (self.res[st.src][1] == 'f16' and MFMA_ROWS_MIN <= R <= MFMA_ROWS_MAX and st.K % 32 == 0
                and st.c0 % 8 == 0 and st.rowlen % 8 == 0):
            return None
        if R > 16 and not self.mfma_ok(c, st, points=False):
            return None
        if -(-P // self.grid) >= MFMA_POINTS_MIN:
            return None
        if name in self.outputs or r in self.private or r in self.outputs or r in self.fx:
            return None
        if list(s[2]) != list(c.reg_axes) + list(st.pts) or list(self.axes_of[r]) != list(s[2]):
            return None
        if not self._additive(c.epi, ('name', '__acc'), '__acc'):
            return None
        if c.A[0] != 'idx' or c.A[1] not in self.axes_of:
            return None
        # point groups of NTS tiles, the fold in KS slices: the fewest bytes per block
        NKB, K = st.K // 32, st.K
        best = None
        for NTS in range(1, (SPLIT_TILES_PACKED if R <= 8 else SPLIT_TILES if R <= 16 else 16) + 1):
            NPG = -(-P // (16 * NTS))
            KS = min(self.grid // NPG, NKB)
            if KS < 2:
                continue
            KSL = -(-NKB // KS)
            cost = R * KSL * 32 * 4 + 16 * NTS * KSL * 32 * 2
            if R > 16:
                # the halves of the block's slice must fit, and every block adds
                # R x its points into the sum (KS adds meet at each address)
                if 2 * R * (KSL * 64 + 16) > MFMA_HALVES_MAX:
                    continue
                cost += R * 16 * NTS * SPLIT_ADD_BYTES
            if best is None or cost < best[0]:
                best = (cost, NTS, NPG, KS, KSL)
        if best is None:
            return None
        _, NTS, NPG, KS, KSL = best
        base = self.rebuild_expr(c.epi, lambda n: ('num', 0.0) if n == ('name', '__acc') else n)
        return dict(c=c, st=st, NTS=NTS, NPG=NPG, KS=KS, KSL=KSL, PG=16 * NTS, base=base,
                    z=self.root(name), axes=list(s[2]))

    def find_splits(self, ss):
        for i, s in enumerate(ss):
            if s[0] == 'step':
                self.find_splits(s[6])
                continue
            sk = self.split_of(s)
            if sk is not None:
                self.splits[id(s)] = sk
                self.fx.add(self.root(s[1]))
                if self.local_folds:
                    sk['p2p'] = self.split_producer(ss, i, s, sk)

    def split_producer(self, ss, i, s, sk):
        """A split whose other factor is the epilogue value g of the stream
        just before it (u; g = EPI(u) at u's points; the split reads g at its
        own points and nothing else reads g): the blocks of a fold slice then
        wait for the blocks that made that slice of g (readiness flags)
        instead of a grid barrier. Returns u's points per block, or None."""
        if i < 2:
            return None
        u, t, c = ss[i - 2], ss[i - 1], sk['c']
        if u[0] != 'let' or t[0] != 'let' or self.place.get(id(u)) not in ('tile', 'lane'):
            return None
        if id(u) in self.splits or id(u) in self.groups or id(u) in self.elided:
            return None
        cu = self.info.get(id(u))
        if getattr(cu, 'kind', None) not in ('tile', 'lane'):
            return None
        stu = self.stream_of(cu)
        if stu is None or len(stu.pts) != 1 or list(stu.pts) != list(c.fold_axes):
            return None
        g = t[1]
        if list(t[2]) != list(u[2]) or top_folds(t[3]) or self.root(g) != g or g in self.private:
            return None
        if g in self.outputs or self.readers_of.get(g, set()) != {id(s)}:
            return None
        if c.A[0] != 'idx' or c.A[1] != g or list(c.A[2]) != [('name', a) for a in t[2]]:
            return None
        P = self.size(stu.pts)
        PPB = -(-P // self.grid)
        NKB, KS = sk['st'].K // 32, sk['KS']
        most = max(((q + 1) * NKB // KS * 32 - 1) // PPB - (q * NKB // KS * 32) // PPB + 1 for q in range(KS))
        if most > 64:
            return None
        return dict(g=g, PPB=PPB)

    def gen_stream_split(self, s, sk, out, ind):
        c, st = sk['c'], sk['st']
        name, z = s[1], self.root(s[1])
        reg = list(c.reg_axes)
        R, P, K, NKB = self.size(reg), self.size(st.pts), st.K, st.K // 32
        NTS, NPG, KS, KSL, PG = sk['NTS'], sk['NPG'], sk['KS'], sk['KSL'], sk['PG']
        NW = self.NWAVE - 1
        RT = 1 if R <= 16 else -(-R // 16)    # row tiles (each tile's accumulators)
        if NTS >= NW:
            TPW, KW = -(-NTS // NW), 1
        else:
            TPW, KW = 1, NW // NTS
        KBW = -(-KSL // KW)
        # the base, everywhere, in the phase before
        self.plan.append((self.show_stmt(s), f'stream (transposed copy) mfma, fold in {KS} slices, '
                          + ('fixed-point sum cleared in the phase before, each slice waiting for the blocks '
                             'that made it' if sk.get('p2p') else 'fixed-point sum: base in the phase before')))
        pp = sk.get('p2p')
        I = ind + '  '
        reads = self.root_reads([c.A]) | {n for n in self.root_reads([s[3]]) if n != z}
        if pp is not None:
            # no grid barrier: z was cleared in the phase before, its base goes
            # in by atomic adds, and each block waits for the makers of its slice
            from .chain import ChainError
            if ((reads - {pp['g']}) & self.dirty) or z in self.readers:
                raise ChainError(f'split {name}: its phase would need a barrier after all')
            self.chain_clear(z, out, ind)
            if not sk.get('base_done'):
                self.chain_base(sk, out, ind)
            PPB, NKB, KS = pp['PPB'], sk['st'].K // 32, sk['KS']
            self.trace.append(('flags', name, frozenset({pp['g']})))
            ranges = [(f'((int)blockIdx.x % {KS} * {NKB} / {KS}) * 32 / {PPB}',
                       f'(((int)blockIdx.x % {KS} + 1) * {NKB} / {KS} * 32 - 1) / {PPB}')]
            active = f'(int)blockIdx.x < {sk["NPG"] * KS}'
            self.trace.append(('flagrange', 'split', ranges, active, (), dict(KS=KS, NKB=NKB, PPB=PPB, grid=self.grid)))
            self.ready_point(name, ranges, active, out, ind, pp['g'])
        else:
            if not sk.get('base_done'):
                self.emit_base(None, z, list(s[2]), sk['base'], out, ind, sync=True)
            self.sync(reads, {z}, out, ind, name)
        sid = self.fresh('k')
        rr, rs = self.rsrc(st.src), self.res_strides(st.src)
        role = [f'const int sg_ = (int)blockIdx.x / {KS}, ss_ = (int)blockIdx.x % {KS};',
                f'const int kb0_ = ss_ * {NKB} / {KS}, nk_ = (ss_ + 1) * {NKB} / {KS} - kb0_;',
                f'const bool mok_ = (int)blockIdx.x < {NPG * KS} && wave < {min(NTS * KW, NW)};',
                f'const int mkp_ = wave / {NTS}, mt_ = wave % {NTS};' if KW > 1 else
                f'const int mkp_ = 0, mt_ = wave;',
                f'const int mk0_ = mkp_ * nk_ / {KW}, mk1_ = (mkp_ + 1) * nk_ / {KW};']

        def tile(i):
            return f'mt_ + {i * NW}' if i else 'mt_'

        def wload(i, kb, dst, cond):
            lines = [f'{{ const int n_ = ({tile(i)}) * 16 + (lane & 15);',
                     f'  const int p_ = sg_ * {PG} + n_;',
                     f'  if (mok_ && ({cond}) && ({tile(i)}) < {NTS} && p_ < {P}) {{']
            env = self.decode('p_', st.pts, lines, '    ', prefix='sp_')
            pre = []
            ix = [self.index(x, env, pre, '    ') for x in st.prefix_idx]
            lines += pre
            base = self.addr(ix, rs[:-1]) if ix else '0'
            lines.append(f'    {dst} = {self.w16("split")}({rr}, (unsigned)({base}) + {st.c0}u + '
                         f'(unsigned)((kb0_ + {kb}) * 32 + (lane >> 4) * 8));')
            lines.append(f'  }} else {dst} = vh_u32x4{{0u, 0u, 0u, 0u}};')
            lines.append('}')
            return lines

        wm = f'wm_{sid}'
        self.decls.append(f'vh_u32x4 {wm}[{TPW}][{KBW}];')

        def make(step_override):
            saved = self.override_step(step_override)
            try:
                lines = [f'if (wave < {NW}) {{'] + ['  ' + x for x in role]
                for i in range(TPW):
                    for j in range(KBW):
                        lines += ['  ' + x for x in wload(i, f'mk0_ + {j}', f'{wm}[{i}][{j}]', f'mk0_ + {j} < mk1_')]
                return lines + ['}']
            finally:
                self.restore_step(saved)
        self.place_prefetch(make, out, ind)
        o = out
        o.append(f'{ind}{{  // stream {name} on the matrix cores, fold in {KS} slices: {P} points x {K} from '
                 f'{st.src}, rows={R}, {PG} points and {KSL} k-blocks per block, waves/tile={KW}')
        o += [I + x for x in role]
        top = self.lds_floats + self.stage_top
        direct = self.direct_lds(c, reg)
        src = None if direct is not None else self.mfma_global_src(c, reg, K)
        if direct is None and src is None:
            if RT > 1:
                raise LowerError(f'split {name}: beyond 16 rows the other factor must be a plain value')
            self.stage_A(c, reg, 0, R, R, K, str(top), o, I)
            direct, top = str(top), top + R * K
        SAB = KSL * 64 + 16
        packed = R <= 8
        ah = top * 4
        al = ah + (8 if packed else R) * SAB
        top = (al + R * SAB) // 4
        red = top
        top += NW * 64 * 4 * RT if KW > 1 else 0
        self.stage_floats = max(self.stage_floats, top - self.lds_floats)
        # the block's slice of the other factor into fp16 halves
        K8 = KSL * 4
        o.append(f'{I}vh_lds_sync();')
        o.append(f'{I}for (int e_ = tid; e_ < {R * K8}; e_ += {self.BLOCK}) {{')
        o.append(f'{I}  const int r_ = e_ / {K8}, k8_ = e_ - r_ * {K8};')
        o.append(f'{I}  float v_[8] = {{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}};')
        o.append(f'{I}  if (k8_ < nk_ * 4) {{')
        o.append(f'{I}    const int col_ = kb0_ * 32 + k8_ * 8;')
        if direct is not None:
            o.append(f'{I}    const float* s_ = sh_f + {direct} + r_ * {K} + col_;')
            o.append(f'{I}    {self.lds_vec_load(8, "s_", "v_")}')
        else:
            o.append(f'{I}    const vh_f32x4 x0_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + col_)), '
                     f'x1_ = ldc4(rb_S, {src}u + (unsigned)(r_ * {K} + col_ + 4));')
            o.append(f'{I}    v_[0] = x0_.x; v_[1] = x0_.y; v_[2] = x0_.z; v_[3] = x0_.w; '
                     f'v_[4] = x1_.x; v_[5] = x1_.y; v_[6] = x1_.z; v_[7] = x1_.w;')
        o.append(f'{I}  }}')
        o.append(f'{I}  vh_u32x4 h_, l_;')
        o.append(f'{I}  {"vh_split8s" if packed else "vh_split8"}(v_, h_, l_);')
        o.append(f'{I}  if (vh_beyond_half8(v_)) stc_u(bar + VH_BAR_ERROR, VH_ERR_RANGE);')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {ah} + r_ * {SAB} + k8_ * 16) = h_;')
        o.append(f'{I}  *(vh_u32x4*)((char*)sh_f + {al} + r_ * {SAB} + k8_ * 16) = l_;')
        o.append(f'{I}}}')
        o.append(f'{I}vh_lds_sync();')
        self.mark(o, I, f'stream {name}: halves')
        if RT == 1:
            o.append(f'{I}vh_f32x4 acc_[{TPW}];')
            o.append(f'{I}#pragma unroll')
            o.append(f'{I}for (int i_ = 0; i_ < {TPW}; ++i_) acc_[i_] = vh_f32x4{{0.f, 0.f, 0.f, 0.f}};')
        else:
            self.mfma_acc_rows(TPW, RT, o, I)
        o.append(f'{I}if (mok_) {{')
        for j in range(KBW):
            if packed:
                o.append(f'{I}  if (mk0_ + {j} < mk1_)')
                o += self.mfma_kstep_packed(f'mk0_ + {j}', lambda i, j=j: f'{wm}[{i}][{j}]', TPW, R, SAB, ah,
                                            I + '    ')
                continue
            o.append(f'{I}  if (mk0_ + {j} < mk1_) {{')
            if RT > 1:
                o += self.mfma_kstep_rows(f'mk0_ + {j}', '', lambda i, j=j: f'{wm}[{i}][{j}]', TPW, RT, R, SAB,
                                          ah, al, I + '    ')
                o.append(f'{I}  }}')
                continue
            o.append(f'{I}    const int ar_ = lane & 15, ak_ = (mk0_ + {j}) * 32 + (lane >> 4) * 8;')
            o.append(f'{I}    const vh_u32x4 ah_ = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {ah} + ar_ * {SAB} '
                     f'+ ak_ * 2) : vh_u32x4{{0u, 0u, 0u, 0u}};')
            o.append(f'{I}    const vh_u32x4 al_ = ar_ < {R} ? *(const vh_u32x4*)((const char*)sh_f + {al} + ar_ * {SAB} '
                     f'+ ak_ * 2) : vh_u32x4{{0u, 0u, 0u, 0u}};')
            for i in range(TPW):
                o.append(f'{I}    acc_[{i}] = vh_mfma(ah_, {wm}[{i}][{j}], acc_[{i}]);')
                o.append(f'{I}    acc_[{i}] = vh_mfma(al_, {wm}[{i}][{j}], acc_[{i}]);')
            o.append(f'{I}  }}')
        o.append(f'{I}}}')
        self.mark(o, I, f'stream {name}: products')
        if KW > 1 and RT > 1:
            self.mfma_parts_rows(KW, NTS, RT, red, o, I)
        elif KW > 1:
            o.append(f'{I}if (mok_ && mkp_ > 0) *(vh_f32x4*)(sh_f + {red} + (wave * 64 + lane) * 4) = acc_[0];')
            o.append(f'{I}vh_lds_sync();')
            o.append(f'{I}if (mok_ && mkp_ == 0) {{')
            for q in range(1, KW):
                o.append(f'{I}  acc_[0] += *(const vh_f32x4*)(sh_f + {red} + ((wave + {q * NTS}) * 64 + lane) * 4);')
            o.append(f'{I}}}')
        # the partial tiles into the fixed-point sum
        o.append(f'{I}if (mok_ && mkp_ == 0) {{')
        if packed:
            o += self.mfma_combine_packed(TPW, I + '  ')
        for i in range(TPW):
            o.append(f'{I}  {{ const int p_ = sg_ * {PG} + ({tile(i)}) * 16 + (lane & 15);')
            o.append(f'{I}    if (({tile(i)}) < {NTS} && p_ < {P}) {{')
            o.append(f'{I}      #pragma unroll')
            o.append(f'{I}      for (int v_ = 0; v_ < 4; ++v_) {{')
            if RT > 1:
                for rt in range(RT):
                    o.append(f'{I}        {{ const int r_ = {rt * 16} + (lane >> 4) * 4 + v_;')
                    o.append(f'{I}          if (r_ < {R}) fxadd(S, {self.gadd(z)} + 2u * (unsigned)(r_ * {P} + p_), '
                             f'acc_[{i}][{rt}][v_]); }}')
                o.append(f'{I}      }}')
                o.append(f'{I}    }}')
                o.append(f'{I}  }}')
                continue
            o.append(f'{I}        const int r_ = (lane >> 4) * 4 + v_;')
            o.append(f'{I}        if (r_ < {R}) fxadd(S, {self.gadd(z)} + 2u * (unsigned)(r_ * {P} + p_), acc_[{i}][v_]);')
            o.append(f'{I}      }}')
            o.append(f'{I}    }}')
            o.append(f'{I}  }}')
        o.append(f'{I}}}')
        o.append(f'{ind}}}')
        self.note(reads, {z})
        self.mark(out, ind, f'stream {name}')
