"""Vesta frontend: source text -> statement list (tuple AST).

This is the half of the reference's ``vesta/interp.py`` that the compiler
needs (lexer ``interp.py:16-31``, expression parser ``:34-90``, statement
parser ``:92-129``). The NumPy evaluator of the reference (``Interp``/``run``,
``interp.py:131-234``) is a CPU path; in this package it has no place on the
GPU path, so ``run`` is not provided here.

AST (the reference's tuple shapes, kept because ``parse`` is public API and
``Lowered.plan`` prints statements):

  expressions  ('num', v) ('name', n) ('neg', e) ('call', f, e)
               ('bin', op, a, b) ('fork', c, a, b) ('idx', name, [e, ...])
               ('fold', op, axis, body)
  statements   ('axis', name, e) ('recv', name, [axes]) ('emit', name, [e, ...], e)
               ('let', name, [axes], e) ('ret', e)
               ('step', name, [axes], var, init, carry, [statements])

Grammar (GRAMMAR.md:19-43 of the reference):

  e    := fork c ? e : e | fold OP AXIS : e | c
  c    := s (== | < | > | <= | >=) s | s
  s    := m ((+|-) m)*        m := u ((*|/) u)*        u := - u | p
  p    := atom [ '[' e, ... ']' ]
  atom := NUMBER | NAME | FUNC '(' e ')' | '(' e ')'
"""
from __future__ import annotations

import re
from dataclasses import dataclass

FOLD_OPS = ('sum', 'max', 'min')
FUNCS = ('exp', 'tanh', 'sqrt')
COMPARE = ('==', '<', '>', '<=', '>=')

# Longest operators first so '<-' is not read as '<' then '-'.
_OPS = ('<-', '->', '==', '<=', '>=', '[', ']', '(', ')', ',', ':', '+', '-', '*', '/', '?', '<', '>', '=')
_NUM = r'\d+\.\d*(?:[eE][-+]?\d+)?|\d+[eE][-+]?\d+|\d+'
_SCAN = re.compile(r'[ \t\r\f\v]*(?:(?P<num>' + _NUM + r')|(?P<name>[A-Za-z_][A-Za-z0-9_]*)|(?P<op>'
                   + '|'.join(re.escape(o) for o in _OPS) + r'))')


@dataclass(frozen=True)
class Token:
    kind: str      # 'num' | 'name' | 'op'
    value: object  # int/float for numbers, str otherwise
    col: int

    def pair(self):
        return (self.kind, self.value)


def tokens(line: str) -> list[Token]:
    """Split one source line (comments already removed) into tokens."""
    out, pos, end = [], 0, len(line.rstrip())
    while pos < end:
        m = _SCAN.match(line, pos)
        if m is None or m.end() == pos:
            raise SyntaxError(f'bad token at {line[pos:end]!r}')
        if m.group('num') is not None:
            text = m.group('num')
            val = float(text) if ('.' in text or 'e' in text or 'E' in text) else int(text)
            out.append(Token('num', val, m.start('num')))
        elif m.group('name') is not None:
            out.append(Token('name', m.group('name'), m.start('name')))
        else:
            out.append(Token('op', m.group('op'), m.start('op')))
        pos = m.end()
    return out


def lex(s: str) -> list[tuple]:
    """(kind, value) pairs, as the reference's ``lex`` returns (interp.py:22-31)."""
    return [t.pair() for t in tokens(s)]


class _Parser:
    """Precedence-climbing expression parser over a token list."""

    def __init__(self, toks: list[Token]):
        self.toks, self.i = toks, 0

    # -- token access
    def at(self, k: int = 0):
        j = self.i + k
        return self.toks[j].value if j < len(self.toks) else None

    def next(self, want=None):
        if self.i >= len(self.toks):
            raise SyntaxError(f'expected {want!r}, got end of line' if want else 'unexpected end of line')
        t = self.toks[self.i]
        if want is not None and t.value != want:
            raise SyntaxError(f'expected {want!r}, got {t.value!r}')
        self.i += 1
        return t

    def finished(self) -> bool:
        return self.i >= len(self.toks)

    # -- grammar
    def expr(self):
        head = self.at()
        if head == 'fork':
            self.next()
            cond = self.compare()
            self.next('?')
            yes = self.expr()
            self.next(':')
            return ('fork', cond, yes, self.expr())
        if head == 'fold' and self.at(1) in FOLD_OPS:
            self.next()
            op = self.next().value
            axis = self.next().value
            self.next(':')
            return ('fold', op, axis, self.expr())
        return self.compare()

    def compare(self):
        lhs = self.binary(0)
        if self.at() in COMPARE:
            op = self.next().value
            return ('bin', op, lhs, self.binary(0))
        return lhs

    _LEVELS = (('+', '-'), ('*', '/'))

    def binary(self, level: int):
        if level == len(self._LEVELS):
            return self.unary()
        lhs = self.binary(level + 1)
        while self.at() in self._LEVELS[level]:
            op = self.next().value
            lhs = ('bin', op, lhs, self.binary(level + 1))
        return lhs

    def unary(self):
        if self.at() == '-':
            self.next()
            return ('neg', self.unary())
        base = self.atom()
        if self.at() == '[':
            self.next()
            idx = [self.expr()]
            while self.at() == ',':
                self.next()
                idx.append(self.expr())
            self.next(']')
            if base[0] != 'name':
                raise SyntaxError('only a name can be indexed')
            base = ('idx', base[1], idx)
        return base

    def atom(self):
        t = self.next()
        if t.kind == 'num':
            return ('num', t.value)
        if t.value == '(':
            e = self.expr()
            self.next(')')
            return e
        if t.kind == 'name':
            if t.value in FUNCS and self.at() == '(':
                self.next('(')
                e = self.expr()
                self.next(')')
                return ('call', t.value, e)
            return ('name', t.value)
        raise SyntaxError(f'unexpected {t.value!r}')

    def name_list(self):
        out = [self.next().value]
        while self.at() == ',':
            self.next()
            out.append(self.next().value)
        return out


def parse_expr(toks):
    """Parse a whole token list as one expression (pairs or Tokens)."""
    if toks and not isinstance(toks[0], Token):
        toks = [Token(k, v, 0) for k, v in toks]
    p = _Parser(list(toks))
    e = p.expr()
    if not p.finished():
        raise SyntaxError(f'trailing {p.at()!r}')
    return e


def _statement(toks: list[Token], line: str):
    """One line -> ('open', stmt) for a step header, ('close',) for end, or ('stmt', stmt)."""
    if line == 'end':
        return ('close',)
    p = _Parser(toks)
    head = toks[0].value
    if head == '->':
        return ('stmt', ('ret', parse_expr(toks[1:])))
    if head == 'axis':
        p.next()
        name = p.next().value
        p.next('=')
        return ('stmt', ('axis', name, parse_expr(toks[p.i:])))
    if head == 'residue':
        p.next()
        name = p.next().value
        if p.finished():
            return ('stmt', ('recv', name, []))
        p.next('[')
        arrow = next((k for k, t in enumerate(toks) if t.value == '<-' and t.kind == 'op'), None)
        if arrow is None:
            return ('stmt', ('recv', name, p.name_list()))
        if toks[arrow - 1].value != ']':
            raise SyntaxError("expected ']' before '<-'")
        inner = _Parser(toks[p.i:arrow - 1])
        idx = [inner.expr()]
        while not inner.finished():
            inner.next(',')
            idx.append(inner.expr())
        return ('stmt', ('emit', name, idx, parse_expr(toks[arrow + 1:])))
    name = p.next().value
    axes = []
    if p.at() == '[':
        p.next()
        axes = p.name_list()
        p.next(']')
    p.next('=')
    if p.at() == 'fold' and p.at(1) == 'step':
        p.next()
        p.next()
        var = p.next().value
        p.next(':')
        rest = toks[p.i:]
        cut = max((k for k, t in enumerate(rest) if t.value == 'as'), default=None)
        if cut is None or cut + 1 >= len(rest):
            raise SyntaxError("fold step needs 'as NAME'")
        return ('open', ('step', name, axes, var, parse_expr(rest[:cut]), rest[cut + 1].value, []))
    return ('stmt', ('let', name, axes, parse_expr(toks[p.i:])))


def parse(text: str) -> list:
    """Program text -> statement list. ``fold step`` blocks nest until ``end``."""
    root: list = []
    open_blocks = [root]
    for lineno, raw in enumerate(text.splitlines(), 1):
        line = raw.split('#', 1)[0].strip()
        if not line:
            continue
        try:
            kind, *rest = _statement(tokens(line), line)
            if kind == 'close':
                if len(open_blocks) == 1:
                    raise SyntaxError("'end' without 'fold step'")
                open_blocks.pop()
            elif kind == 'open':
                open_blocks[-1].append(rest[0])
                open_blocks.append(rest[0][6])
            else:
                open_blocks[-1].append(rest[0])
        except SyntaxError as err:
            raise SyntaxError(f'line {lineno}: {raw.strip()!r}: {err}') from None
    if len(open_blocks) != 1:
        raise SyntaxError('missing end')
    return root
