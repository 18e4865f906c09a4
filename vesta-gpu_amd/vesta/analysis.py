"""Front half of the gfx950 lowering: facts about a program and the rewrites
that run before placement (batch lift, normalisation, hoisting, aliasing,
inlining), plus the expression queries the placement and code generation
ask of it.

Every pass here is a small rule over two shared tools: the table-driven tree
helpers of ``vesta.ir`` (so no pass spells out the node kinds it does not
touch) and ``DefUse``, one index of where each named value is defined and
read. The rules themselves are the language's (``GRAMMAR.md`` of the
reference: named axes, folds remove their axis, an emit is visible to later
reads, a step carries a value through its loop) and the compiler's own
placement policy; what each decides is stated at the rule.

Reference behaviour these passes agree with (same statement plan for the
GPT-2 program): batch lift ``vesta/lower.py:109-132``; hoist, alias, inline
``vesta/lower.py:187-310``; the private-placement test ``vesta/lower.py:357-367``.
"""
from __future__ import annotations

import math
from collections import Counter

from .ir import (STEP_BODY, at_axes, defined_names, is_node, kids, map_stmt, outermost, statements, stmt_exprs,
                 substitute, transform, walk)

BIG = 1 << 16                 # a residue this large is streamed, never recomputed per point
PRIV_SIZE = 8192              # a private value holds at most this many floats
PRIV_WORK = 1 << 17           # ... and costs at most this many operations per block
STAGE_MAX = 8192              # a private statement reads at most this many floats of locals


class LowerError(ValueError):
    pass


def is_fold(n):
    return n[0] == 'fold'


def top_folds(e):
    """Folds of ``e`` not inside another fold."""
    return outermost(e, is_fold)


def replace_node(e, target, repl):
    """``e`` with the node ``target`` (by identity) replaced by ``repl``."""
    return substitute(e, {id(target): repl})


def map_program(stmts, expr_fn, header=None):
    """Apply ``expr_fn`` to every expression of every statement, descending
    into step bodies. ``header(s)`` may then rewrite a statement's own
    non-expression fields (it gets the statement with its expressions and
    body already mapped)."""
    out = []
    for s in stmts:
        t = map_stmt(s, expr_fn)
        if t[0] == 'step':
            t = t[:STEP_BODY] + (map_program(t[STEP_BODY], expr_fn, header),) + t[STEP_BODY + 1:]
        out.append(header(t) if header else t)
    return out


def batch_lift(stmts, B, per_token, bax='bt'):
    """Ask the program of B tokens at once: an axis ``bax`` of extent B is
    declared first, and it becomes the leading axis of every value the program
    defines and of every per-token residue (its reads gain a leading ``bax``
    index; an emit into it writes at the token's row). Residues that are the
    same for every token keep their shape. Same meaning as reference
    ``vesta/lower.py:109-132``."""
    own = defined_names(stmts)
    per_token = set(per_token)

    def row():
        return ('name', bax)          # a fresh node per use: later passes key nodes by identity

    def lift_read(n):
        k = n[0]
        if k == 'name' and n[1] in per_token and n[1] not in own:
            return ('idx', n[1], [row()])                # a per-token scalar residue
        if k == 'idx' and (n[1] in own or n[1] in per_token):
            return ('idx', n[1], [row(), *n[2]])
        return n

    def lift_header(s):
        k = s[0]
        if k in ('let', 'step'):
            return s[:2] + ([bax, *s[2]],) + s[3:]
        if k == 'emit' and s[1] in per_token:
            return (k, s[1], [row(), *s[2]], s[3])
        return s

    body = map_program(stmts, lambda e: transform(e, lift_read), lift_header)
    return [('axis', bax, ('num', B))] + body


class DefUse:
    """Where named values are defined and read in a statement list (step
    bodies included): ``defs`` name -> its let statement, ``uses`` name ->
    number of reads, ``readers`` name -> ids of the statements reading it."""

    def __init__(self, stmts, is_value):
        self.defs, self.uses, self.readers = {}, Counter(), {}
        for s in statements(stmts):
            if s[0] == 'let':
                self.defs[s[1]] = s
            for e in stmt_exprs(s):
                for n in walk(e):
                    if n[0] in ('name', 'idx') and is_value(n[1]):
                        self.uses[n[1]] += 1
                        self.readers.setdefault(n[1], set()).add(id(s))


class Analysis:
    """Program facts and pre-placement rewrites (mixed into ``Lowering``)."""

    # ------------------------------------------------------------ facts
    def scan(self, ss):
        """Record axis extents (upper bounds for those set at run time), the
        axes of every defined value, step variables and emitted residues."""
        for s in statements(ss):
            kind = s[0]
            if kind == 'axis':
                name, ext = s[1], s[2]
                if ext[0] == 'num':
                    self.static[name] = int(ext[1])
                    continue
                if name not in self.axis_max:
                    raise LowerError(f'axis {name} is set at run time: give its upper bound in axis_max')
                self.static[name] = int(self.axis_max[name])
                self.dynamic[name] = ext
            elif kind in ('recv', 'emit') and s[1] not in self.res:
                raise NameError(f'residue {s[1]} not supplied')
            elif kind == 'let':
                self.axes_of[s[1]] = tuple(s[2])
            elif kind == 'step':
                self.steps.add(s[3])
                for n in (s[1], s[5]):
                    self.axes_of[n] = tuple(s[2])
            if kind == 'emit':
                self.emitted.add(s[1])
                self.emit_stmts.append(s)

    def is_axis(self, n):
        return n in self.static and n not in self.steps

    def ext_c(self, a):
        """C expression of an axis extent."""
        return f'E_{a}' if a in self.dynamic else str(self.static[a])

    def size(self, axes):
        return math.prod(self.static[a] for a in axes)

    def is_value(self, n):
        """A name the program computes or emits (as opposed to an axis or a
        read-only residue)."""
        return n in self.axes_of or n in self.emitted

    # ------------------------------------------------------------ queries
    def free_axes(self, e):
        """Axes ``e`` varies along outside its own folds."""
        k = e[0]
        if k == 'name':
            return {e[1]} if self.is_axis(e[1]) else set(self.axes_of.get(e[1], ()))
        if k == 'fold':
            return self.free_axes(e[3]) - {e[2]}
        acc = set()
        for n in (e[2] if k == 'idx' else e[1:]):
            if is_node(n):
                acc |= self.free_axes(n)
        return acc

    def reads(self, e):
        """Values (locals and emitted residues) ``e`` reads."""
        return {n[1] for n in walk(e) if n[0] in ('name', 'idx') and self.is_value(n[1])}

    def res_reads(self, e):
        return [n for n in walk(e) if n[0] == 'idx' and n[1] in self.res]

    def big_reads(self, e):
        """Reads of large read-only residues (weights): streamed, never recomputed."""
        return [n for n in self.res_reads(e) if n[1] not in self.emitted and math.prod(self.res[n[1]][0]) > BIG]

    def fold_work(self, e):
        """Inner-loop trip count of ``e`` per output point (nested folds multiply)."""
        best = 1
        stack = [(e, 1)]
        while stack:
            n, mult = stack.pop()
            if not is_node(n):
                continue
            if n[0] == 'fold':
                mult *= self.static[n[2]]
                best = max(best, mult)
                stack.append((n[3], mult))
            else:
                stack.extend((k, mult) for k in kids(n))
        return best

    def root(self, n):
        """The storage a value finally lives in, following aliases."""
        seen = n
        while seen in self.alias:
            seen = self.alias[seen]
        return seen

    def big_contraction(self, s):
        return s[0] == 'let' and any(self.big_reads(f[3]) for f in top_folds(s[3]))

    # ------------------------------------------------------------ rewrites
    def normalise(self, ss):
        """A bare read of a value that has axes reads it at its own axes."""
        def at_own(n):
            if n[0] == 'name' and self.axes_of.get(n[1]):
                return at_axes(n[1], self.axes_of[n[1]])
            return n
        return map_program(ss, lambda e: transform(e, at_own))

    def hoist(self, ss):
        """A fold that varies along only some (or none) of its statement's axes
        is computed once per point of those, as a statement of its own placed
        just before (the softmax denominator: once per (bt, h), not per s).
        Hoisted values are named ``_h1``, ``_h2``, ... in program order."""
        out = []
        for s in ss:
            if s[0] == 'step':
                out.append(s[:STEP_BODY] + (self.hoist(s[STEP_BODY]),))
                continue
            if s[0] != 'let':
                out.append(s)
                continue
            axes = list(s[2])
            want, repl = set(axes), {}
            for f in top_folds(s[3]):
                free = self.free_axes(f)
                if not free < want:            # needs every axis, or one the statement lacks
                    continue
                self.tmp += 1
                name = f'_h{self.tmp}'
                kept = [a for a in axes if a in free]
                self.axes_of[name] = tuple(kept)
                out.append(('let', name, kept, f))
                repl[id(f)] = at_axes(name, kept)
            out.append(('let', s[1], axes, substitute(s[3], repl) if repl else s[3]))
        return out

    def find_aliases(self, ss):
        """Storage sharing around step loops. A step's result always lives in
        its carry. The value a loop starts from (``init``) or hands back
        (``ret``) lives there too when nothing else needs it separately: it is
        a plain read, at its own axes, of a value read exactly once, with the
        loop's axes, whose definition does not read the carry, and which the
        host does not ask for."""
        du = DefUse(ss, self.is_value)

        def shares(e, axes, carry):
            if e[0] != 'idx' or e[1] not in du.defs or du.uses[e[1]] != 1:
                return False
            own = self.axes_of[e[1]]
            return (own == tuple(axes) and e[2] == [('name', a) for a in own]
                    and carry not in self.reads(du.defs[e[1]][3]) and e[1] not in self.outputs)

        for s in statements(ss):
            if s[0] != 'step':
                continue
            _, name, axes, _var, init, carry, body = s
            rets = [b for b in body if b[0] == 'ret']
            if len(rets) != 1:
                raise SyntaxError(f'step {name} needs exactly one ->')
            for e in (init, rets[0][1]):
                if shares(e, axes, carry):
                    self.alias[e[1]] = carry
            self.alias[name] = carry

    def inline(self, ss):
        """A value computed without a fold is not stored: its expression is
        substituted where it is read, provided every reader is a later plain
        statement (let or emit) that does not stream a weight through a fold
        (re-evaluating it inside that loop would multiply its cost), and the
        value is not asked for by the host, aliased, or a loop carry."""
        out = [s[:STEP_BODY] + (self.inline(s[STEP_BODY]),) if s[0] == 'step' else s for s in ss]
        carries = set(self.alias.values())
        i = 0
        while i < len(out):
            s = out[i]
            name = s[1] if s[0] == 'let' else None
            if name is None or top_folds(s[3]) or name in self.outputs or name in self.alias or name in carries:
                i += 1
                continue
            later = out[i + 1:]
            readers = [t for t in later if any(name in self.reads(e)
                                               for u in statements([t]) for e in stmt_exprs(u))]
            if not readers or any(t[0] not in ('let', 'emit') or self.big_contraction(t) for t in readers):
                i += 1
                continue
            axes, body = list(s[2]), s[3]

            def expand(n, name=name, axes=axes, body=body):
                if n[0] == 'name' and n[1] == name:
                    return body
                if n[0] == 'idx' and n[1] == name:
                    at = dict(zip(axes, n[2]))
                    return transform(body, lambda m: at.get(m[1], m) if m[0] == 'name' else m)
                return n
            out[i + 1:] = [map_stmt(t, lambda e: transform(e, expand)) if t[0] in ('let', 'emit') else t
                           for t in later]
            del out[i]
            self.inlined.append(name)
        return out

    # ------------------------------------------------------------ placement entry
    def place_all(self, ss):
        self.place = {}           # id(stmt) -> placement string
        self.info = {}            # id(stmt) -> Contraction / extra info
        self.groups = {}          # id(first stmt) -> (lead axes, [stmts])
        self.in_group = set()
        self.private = set()
        self.argmax = {}          # id(max statement) -> the lowest-index statement that reads it
        self.group_local = {}     # id(first stmt of a group) -> names kept in LDS
        self.readers_of = DefUse(ss, self.is_value).readers   # name -> ids of statements reading it
        self._place_block(ss)

    def priv_ok(self, s):
        """Can every block compute statement ``s`` for itself (in LDS)? Only a
        small value, cheap per block, over static axes, whose inputs are small
        locals or small read-only residues, and which no loop or host keeps."""
        name = s[1]
        if name in self.outputs or name in self.alias or name in set(self.alias.values()):
            return False
        points = self.size(s[2])
        if points > PRIV_SIZE or points * self.fold_work(s[3]) > PRIV_WORK:
            return False
        if any(a in self.dynamic for a in s[2]):
            return False
        staged = sum(self.size(self.axes_of[n]) for n in self.reads(s[3])
                     if n in self.axes_of and n not in self.private)
        if staged > STAGE_MAX:
            return False
        return all(n[1] not in self.emitted and math.prod(self.res[n[1]][0]) <= BIG for n in self.res_reads(s[3]))
