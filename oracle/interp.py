"""ORACLE -- test infrastructure, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or the CPU baseline that
is timed beside the GPU). The GPU path never calls it.

A CPU restatement of the reference NumPy interpreter ``vesta/interp.py``:

  lexer            interp.py:16-31
  expression parse interp.py:34-90
  statement parse  interp.py:92-129
  evaluation       interp.py:131-234  (align :139-147, ev :153-188,
                   contract :190-198, fill :200-203, exec :205-231, run :233)

It has its own lexer and parser, written apart from the product frontend,
so a parser mistake in one is caught by the AST comparison against the other.

Numerics follow the reference operation for operation, because the reference
interpreter's exact fp32 results are the contract for greedy tokens:
  * every named value carries its axis names; operands line up by name
    (GRAMMAR.md:50), absent axes broadcast as size 1 (interp.py:139-147);
  * ``fold sum`` whose body is a product is one ``np.einsum(..., optimize=True)``
    over the two factors (interp.py:183-184, :190-198); every other fold is
    ``np.sum/np.max/np.min`` along the axis (interp.py:185-187);
  * ``fork`` is ``np.where``; indexing is NumPy fancy indexing on index arrays
    broadcast over the union of their axes (interp.py:174-180);
  * an emit writes into the residue array in place, so an fp16 residue rounds
    the value to fp16 (round to nearest even) (interp.py:212-218);
  * ``fold step`` is a Python loop carrying the value (interp.py:221-231).

Parity: pinned by the golden vectors in tests/golden (written by importing
the reference interpreter in the build container), by a brute-force
pure-Python GPT-2 on tiny shapes and by a textbook NumPy GPT-2.
"""
import re

import numpy as np

# ------------------------------------------------------------------ lexing
_TOKEN = re.compile(
    r'\s*(?:(?P<n>\d+\.\d*(?:[eE][-+]?\d+)?|\d+[eE][-+]?\d+|\d+)'
    r'|(?P<w>[A-Za-z_]\w*)'
    r'|(?P<o><-|->|==|<=|>=|[\[\](),:+\-*/?<>=]))')

_REDUCE = {'sum': np.sum, 'max': np.max, 'min': np.min}
_UNARY = {'exp': np.exp, 'tanh': np.tanh, 'sqrt': np.sqrt}
_BINARY = {'+': np.add, '-': np.subtract, '*': np.multiply, '/': np.divide,
           '==': np.equal, '<': np.less, '>': np.greater, '<=': np.less_equal, '>=': np.greater_equal}
_CMP = ('==', '<', '>', '<=', '>=')


def lex(line):
    """Tokens of one line as (kind, value); kind is 'num', 'name' or 'op'."""
    line = line.rstrip()
    out, pos = [], 0
    while pos < len(line):
        m = _TOKEN.match(line, pos)
        if m is None or m.end() == pos:
            raise SyntaxError(f'bad token at {line[pos:]!r}')
        if m.group('n') is not None:
            txt = m.group('n')
            out.append(('num', float(txt) if any(ch in txt for ch in '.eE') else int(txt)))
        elif m.group('w') is not None:
            out.append(('name', m.group('w')))
        else:
            out.append(('op', m.group('o')))
        pos = m.end()
    return out


# ------------------------------------------------------------------ parsing
class _Cursor:
    def __init__(self, toks):
        self.toks = toks
        self.k = 0

    def look(self, ahead=0):
        j = self.k + ahead
        return self.toks[j][1] if j < len(self.toks) else None

    def eat(self, want=None):
        tok = self.toks[self.k] if self.k < len(self.toks) else (None, None)
        if want is not None and tok[1] != want:
            raise SyntaxError(f'expected {want!r}, got {tok[1]!r}')
        self.k += 1
        return tok

    def empty(self):
        return self.k >= len(self.toks)


def _expr(c):
    if c.look() == 'fork':
        c.eat()
        test = _cmp(c)
        c.eat('?')
        a = _expr(c)
        c.eat(':')
        return ('fork', test, a, _expr(c))
    if c.look() == 'fold' and c.look(1) in _REDUCE:
        c.eat()
        op = c.eat()[1]
        ax = c.eat()[1]
        c.eat(':')
        return ('fold', op, ax, _expr(c))
    return _cmp(c)


def _cmp(c):
    a = _sum(c)
    if c.look() in _CMP:
        op = c.eat()[1]
        return ('bin', op, a, _sum(c))
    return a


def _sum(c):
    a = _prod(c)
    while c.look() in ('+', '-'):
        op = c.eat()[1]
        a = ('bin', op, a, _prod(c))
    return a


def _prod(c):
    a = _neg(c)
    while c.look() in ('*', '/'):
        op = c.eat()[1]
        a = ('bin', op, a, _neg(c))
    return a


def _neg(c):
    if c.look() == '-':
        c.eat()
        return ('neg', _neg(c))
    a = _atom(c)
    if c.look() == '[':
        c.eat()
        ix = [_expr(c)]
        while c.look() == ',':
            c.eat()
            ix.append(_expr(c))
        c.eat(']')
        a = ('idx', a[1], ix)
    return a


def _atom(c):
    kind, v = c.eat()
    if kind == 'num':
        return ('num', v)
    if v == '(':
        e = _expr(c)
        c.eat(')')
        return e
    if kind == 'name' and v in _UNARY and c.look() == '(':
        c.eat('(')
        e = _expr(c)
        c.eat(')')
        return ('call', v, e)
    if kind == 'name':
        return ('name', v)
    raise SyntaxError(f'unexpected {v!r}')


def parse_expr(toks):
    c = _Cursor(toks)
    e = _expr(c)
    if not c.empty():
        raise SyntaxError(f'trailing {c.look()!r}')
    return e


def parse(text):
    """Program text -> statement list (same tuple shapes as the reference)."""
    top = []
    blocks = [top]
    for lineno, raw in enumerate(text.splitlines(), 1):
        line = raw.split('#', 1)[0].strip()
        if not line:
            continue
        try:
            toks = lex(line)
            body = blocks[-1]
            if line == 'end':
                blocks.pop()
                continue
            first = toks[0][1]
            if first == '->':
                body.append(('ret', parse_expr(toks[1:])))
                continue
            c = _Cursor(toks)
            if first == 'axis':
                c.eat()
                nm = c.eat()[1]
                c.eat('=')
                body.append(('axis', nm, parse_expr(toks[c.k:])))
                continue
            if first == 'residue':
                c.eat()
                nm = c.eat()[1]
                if c.empty():
                    body.append(('recv', nm, []))
                    continue
                c.eat('[')
                if ('op', '<-') not in toks:
                    names = [c.eat()[1]]
                    while c.look() == ',':
                        c.eat()
                        names.append(c.eat()[1])
                    body.append(('recv', nm, names))
                    continue
                arrow = toks.index(('op', '<-'))
                inner = _Cursor(toks[c.k:arrow - 1])
                ix = [_expr(inner)]
                while not inner.empty():
                    inner.eat(',')
                    ix.append(_expr(inner))
                body.append(('emit', nm, ix, parse_expr(toks[arrow + 1:])))
                continue
            nm = c.eat()[1]
            axes = []
            if c.look() == '[':
                c.eat()
                axes = [c.eat()[1]]
                while c.look() == ',':
                    c.eat()
                    axes.append(c.eat()[1])
                c.eat(']')
            c.eat('=')
            if c.look() == 'fold' and c.look(1) == 'step':
                c.eat()
                c.eat()
                var = c.eat()[1]
                c.eat(':')
                rest = toks[c.k:]
                cut = max(i for i, t in enumerate(rest) if t[1] == 'as')
                block = []
                body.append(('step', nm, axes, var, parse_expr(rest[:cut]), rest[cut + 1][1], block))
                blocks.append(block)
                continue
            body.append(('let', nm, axes, parse_expr(toks[c.k:])))
        except SyntaxError as err:
            raise SyntaxError(f'line {lineno}: {raw.strip()!r}: {err}') from None
    if len(blocks) != 1:
        raise SyntaxError('missing end')
    return top


# ------------------------------------------------------------------ evaluation
def _merge(*axis_lists):
    """Union of axis names, first-seen order (interp.py:132-137)."""
    seen = []
    for axes in axis_lists:
        for a in axes:
            if a not in seen:
                seen.append(a)
    return tuple(seen)


def _lay_out(val, axes, target):
    """Put val (with axes) on target's axis order, size 1 where absent (interp.py:139-147)."""
    if not axes:
        return val
    arr = np.asarray(val).transpose([axes.index(a) for a in target if a in axes])
    dims, src = [], iter(arr.shape)
    for a in target:
        dims.append(next(src) if a in axes else 1)
    return arr.reshape(dims)


class Machine:
    """Evaluates a statement list against a residue dict (interp.py:149-231).

    ``fast=True`` replaces a fancy-index gather whose indices are all scalars
    or distinct plain axes (``qkvw[l, d, j]``, ``wte[n, d]``) by a basic slice
    (a view when it is already C-contiguous and 64-byte aligned, else a fresh
    C-contiguous copy): the same values, shape, dtype and layout as the
    gather, many times faster. ``fast=False`` is the reference
    behaviour; the tests check the two give identical bits.
    """

    def __init__(self, residue, fast=False):
        self.res = residue
        self.env = {}
        self.ext = {}
        self.fast = fast

    # expressions ---------------------------------------------------------
    def value(self, e):
        return getattr(self, '_v_' + e[0])(e)

    def _v_num(self, e):
        return e[1], ()

    def _v_name(self, e):
        n = e[1]
        if n in self.env:
            return self.env[n]
        if n in self.ext:
            return np.arange(self.ext[n]), (n,)
        if n in self.res and np.ndim(self.res[n]) == 0:
            return self.res[n], ()
        raise NameError(n)

    def _v_neg(self, e):
        v, ax = self.value(e[1])
        return -v, ax

    def _v_call(self, e):
        v, ax = self.value(e[2])
        return _UNARY[e[1]](v), ax

    def _v_bin(self, e):
        a, aa = self.value(e[2])
        b, ba = self.value(e[3])
        u = _merge(aa, ba)
        return _BINARY[e[1]](_lay_out(a, aa, u), _lay_out(b, ba, u)), u

    def _v_fork(self, e):
        (c, ca), (a, aa), (b, ba) = (self.value(x) for x in e[1:])
        u = _merge(ca, aa, ba)
        return np.where(_lay_out(c, ca, u), _lay_out(a, aa, u), _lay_out(b, ba, u)), u

    def _v_idx(self, e):
        name = e[1]
        if self.fast:
            sliced = self._slice_copy(e)
            if sliced is not None:
                return sliced
        parts = [self.value(x) for x in e[2]]
        src = self.env[name][0] if name in self.env else self.res[name]
        u = _merge(*[ax for _, ax in parts])
        shape = tuple(self.ext.get(a, 1) for a in u)
        if u:
            index = tuple(np.broadcast_to(_lay_out(v, ax, u), shape) for v, ax in parts)
        else:
            index = tuple(v for v, _ in parts)
        return src[index], u

    def _slice_copy(self, e):
        """Basic-slice form of an index whose parts are scalars or distinct plain axes."""
        src = self.env[e[1]][0] if e[1] in self.env else self.res[e[1]]
        index, axes = [], []
        for x in e[2]:
            if x[0] == 'name' and x[1] not in self.env and x[1] in self.ext:
                if x[1] in axes:
                    return None
                axes.append(x[1])
                index.append(slice(0, self.ext[x[1]]))
                continue
            v, ax = self.value(x)
            if ax:
                return None
            index.append(v)
        if not axes:
            return None
        view = np.asarray(src)[tuple(index)]
        if view.flags.c_contiguous and view.ctypes.data % 64 == 0:
            return view, tuple(axes)       # already laid out as a fresh gather would be
        return np.array(view, order='C', copy=True), tuple(axes)

    def _v_fold(self, e):
        op, axis, body = e[1], e[2], e[3]
        if op == 'sum' and body[0] == 'bin' and body[1] == '*':
            return self._contract(axis, body[2], body[3])
        v, ax = self.value(body)
        if axis not in ax:
            raise ValueError(f'fold over {axis} but body has axes {ax}')
        return _REDUCE[op](v, axis=ax.index(axis)), tuple(a for a in ax if a != axis)

    def _contract(self, axis, left, right):
        (a, aa), (b, ba) = self.value(left), self.value(right)
        u = _merge(aa, ba)
        if axis not in u:
            raise ValueError(f'fold over {axis} but body has axes {u}')
        letter = {n: chr(ord('a') + i) for i, n in enumerate(u)}
        keep = tuple(n for n in u if n != axis)
        spec = '{},{}->{}'.format(''.join(letter[n] for n in aa), ''.join(letter[n] for n in ba),
                                  ''.join(letter[n] for n in keep))
        return np.einsum(spec, np.asarray(a), np.asarray(b), optimize=True), keep

    # statements ----------------------------------------------------------
    def _shaped(self, v, ax, lhs):
        """Broadcast a value onto its left-side axes (interp.py:200-203)."""
        if not set(ax) <= set(lhs):
            raise ValueError(f'value has axes {ax}, left side only {lhs}')
        if not lhs:
            return v
        return np.array(np.broadcast_to(_lay_out(v, ax, lhs), tuple(self.ext[a] for a in lhs)))

    def run_block(self, stmts):
        for s in stmts:
            kind = s[0]
            if kind == 'axis':
                self.ext[s[1]] = int(self.value(s[2])[0])
            elif kind == 'recv':
                if s[1] not in self.res:
                    raise NameError(f'residue {s[1]} not supplied')
            elif kind == 'emit':
                parts = [self.value(x) for x in s[2]]
                v, ax = self.value(s[3])
                u = _merge(*[a for _, a in parts])
                if not set(ax) <= set(u):
                    raise ValueError(f'emit value has axes {ax}, index only {u}')
                shape = tuple(self.ext[a] for a in u)
                if u:
                    index = tuple(np.broadcast_to(_lay_out(i, a, u), shape) for i, a in parts)
                    self.res[s[1]][index] = np.broadcast_to(_lay_out(v, ax, u), shape)
                else:
                    self.res[s[1]][tuple(i for i, _ in parts)] = v
            elif kind == 'let':
                v, ax = self.value(s[3])
                self.env[s[1]] = (self._shaped(v, ax, s[2]), tuple(s[2]))
            elif kind == 'step':
                _, name, lhs, var, init, carry, block = s
                rets = [b for b in block if b[0] == 'ret']
                if len(rets) != 1:
                    raise SyntaxError(f'step {name} needs exactly one ->')
                body = [b for b in block if b[0] != 'ret']
                cur = (self._shaped(*self.value(init), lhs), tuple(lhs))
                for i in range(self.ext[var]):
                    self.env[var] = (i, ())
                    self.env[carry] = cur
                    self.run_block(body)
                    cur = (self._shaped(*self.value(rets[0][1]), lhs), tuple(lhs))
                del self.env[var]
                self.env[name] = cur
            # a 'ret' outside a step block is ignored, as in interp.py:205-231


def run(text, residue, fast=False):
    """Run a program; emits write into ``residue``; returns the env (interp.py:233-234)."""
    m = Machine(residue, fast=fast)
    m.run_block(parse(text))
    return m.env
