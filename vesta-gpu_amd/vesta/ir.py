"""Program trees as the parser builds them, and one generic way to visit and
rewrite them.

Expressions are tuples whose first field names the kind:

    ('num', value)            ('name', n)            ('idx', n, [index, ...])
    ('fold', op, axis, body)  ('neg', x)             ('call', fn, x)
    ('bin', op, a, b)         ('fork', cond, a, b)

Statements likewise: ('axis', n, extent), ('recv', n, ...), ('let', n, axes,
value), ('emit', residue, [index, ...], value), ('step', n, axes, var, init,
carry, [statement, ...]), ('ret', value).

Instead of a hand-written case per kind in every pass, each kind lists which
of its fields hold sub-expressions (``EXPR_FIELDS`` / ``STMT_FIELDS``); the
helpers below read those tables, so a pass states only what it does at the
nodes it cares about.
"""
from __future__ import annotations

ONE, MANY = 'one', 'many'

EXPR_FIELDS = {
    'num': (),
    'name': (),
    'idx': ((2, MANY),),
    'fold': ((3, ONE),),
    'neg': ((1, ONE),),
    'call': ((2, ONE),),
    'bin': ((2, ONE), (3, ONE)),
    'fork': ((1, ONE), (2, ONE), (3, ONE)),
}

STMT_FIELDS = {
    'axis': ((2, ONE),),
    'recv': (),
    'let': ((3, ONE),),
    'emit': ((2, MANY), (3, ONE)),
    'step': ((4, ONE),),
    'ret': ((1, ONE),),
}
STEP_BODY = 6        # field of a step statement holding its statements


def is_node(e) -> bool:
    return isinstance(e, tuple) and bool(e) and isinstance(e[0], str)


def _fields(e, table):
    return table.get(e[0], ())


def kids(e):
    """The direct sub-expressions of an expression node, in field order."""
    for pos, kind in _fields(e, EXPR_FIELDS):
        if kind == ONE:
            yield e[pos]
        else:
            yield from e[pos]


def with_kids(e, fn, table=EXPR_FIELDS):
    """A copy of node ``e`` whose sub-expression fields hold ``fn`` of the old ones."""
    spec = _fields(e, table)
    if not spec:
        return e
    parts = list(e)
    for pos, kind in spec:
        parts[pos] = fn(parts[pos]) if kind == ONE else [fn(x) for x in parts[pos]]
    return tuple(parts)


def walk(e):
    """Every expression node of ``e``, each before its sub-expressions, left to right."""
    if not is_node(e):
        return
    stack = [e]
    while stack:
        n = stack.pop()
        yield n
        ks = [k for k in kids(n) if is_node(k)]
        stack.extend(reversed(ks))


def transform(e, post):
    """Rewrite bottom-up: sub-expressions first, then ``post`` of the rebuilt node."""
    if not is_node(e):
        return e
    return post(with_kids(e, lambda k: transform(k, post)))


def substitute(e, repl: dict):
    """``e`` with every node whose id is a key of ``repl`` replaced by its value
    (the replacement is not visited again)."""
    if not is_node(e):
        return e
    hit = repl.get(id(e))
    if hit is not None:
        return hit
    return with_kids(e, lambda k: substitute(k, repl))


def outermost(e, pred):
    """Nodes of ``e`` satisfying ``pred`` that no other such node contains."""
    found, stack = [], [e] if is_node(e) else []
    while stack:
        n = stack.pop()
        if pred(n):
            found.append(n)
            continue
        stack.extend(reversed([k for k in kids(n) if is_node(k)]))
    return found


def stmt_exprs(s):
    """The expressions held by a statement's own fields (not its body)."""
    out = []
    for pos, kind in _fields(s, STMT_FIELDS):
        if kind == ONE:
            out.append(s[pos])
        else:
            out.extend(s[pos])
    return out


def map_stmt(s, fn):
    """A copy of statement ``s`` with ``fn`` applied to each of its expressions
    (a step's body is left as it is)."""
    return with_kids(s, fn, STMT_FIELDS)


def statements(stmts):
    """Every statement, a step before the statements of its body."""
    for s in stmts:
        yield s
        if s[0] == 'step':
            yield from statements(s[STEP_BODY])


def defined_names(stmts, into=None) -> set:
    """Names the program defines: lets, steps and their carries, at any depth."""
    into = set() if into is None else into
    for s in statements(stmts):
        if s[0] == 'let':
            into.add(s[1])
        elif s[0] == 'step':
            into.update((s[1], s[5]))
    return into


def axis_ref(a):
    return ('name', a)


def at_axes(name, axes):
    """A read of ``name`` at the index list ``axes`` (a scalar read when empty)."""
    return ('idx', name, [axis_ref(a) for a in axes]) if axes else ('name', name)
