"""Product frontend (vesta.interp): lexing and parsing to the reference's tuple AST.

The oracle has its own parser (oracle/interp.py); the two must agree on every
program, and the reference program text must parse to the same AST as this
repository's gpt2.vst (reference vesta/programs/gpt2.vst:1-82)."""
import os

import pytest

from oracle import interp as oracle
from vesta import interp as fe
from vesta.gpt2_program import gpt2_program

from conftest import PKG, REFERENCE

PROGRAMS = os.path.join(PKG, 'vesta', 'programs')


def test_lex_kinds():
    assert fe.lex('a[i] <- 1.5e-3 * b2 >= 7') == [
        ('name', 'a'), ('op', '['), ('name', 'i'), ('op', ']'), ('op', '<-'), ('num', 1.5e-3), ('op', '*'),
        ('name', 'b2'), ('op', '>='), ('num', 7)]
    assert fe.lex('3.') == [('num', 3.0)] and fe.lex('2e3') == [('num', 2000.0)] and fe.lex('12') == [('num', 12)]


def test_lex_rejects_bad_token():
    with pytest.raises(SyntaxError):
        fe.lex('a $ b')


def test_precedence_and_forms():
    e = fe.parse_expr(fe.lex('fork a - b * -c < d ? fold max i: x[i] : 2 / y'))
    assert e == ('fork', ('bin', '<', ('bin', '-', ('name', 'a'), ('bin', '*', ('name', 'b'), ('neg', ('name', 'c')))),
                          ('name', 'd')),
                 ('fold', 'max', 'i', ('idx', 'x', [('name', 'i')])),
                 ('bin', '/', ('num', 2), ('name', 'y')))
    assert fe.parse_expr(fe.lex('exp(a) + tanh(b[i, j * 2])')) == (
        'bin', '+', ('call', 'exp', ('name', 'a')), ('call', 'tanh', ('idx', 'b', [('name', 'i'), ('bin', '*', ('name', 'j'), ('num', 2))])))


def test_statements():
    prog = fe.parse('''
axis n = 4          # comment
residue w[n]
residue y
residue k[n, n] <- w[n] * 2
z[n] = fold step i: w as c
    q[n] = c[n] + 1
    -> q
end
''')
    assert prog[0] == ('axis', 'n', ('num', 4))
    assert prog[1] == ('recv', 'w', ['n']) and prog[2] == ('recv', 'y', [])
    assert prog[3] == ('emit', 'k', [('name', 'n'), ('name', 'n')], ('bin', '*', ('idx', 'w', [('name', 'n')]), ('num', 2)))
    assert prog[4][:6] == ('step', 'z', ['n'], 'i', ('name', 'w'), 'c')
    assert prog[4][6] == [('let', 'q', ['n'], ('bin', '+', ('idx', 'c', [('name', 'n')]), ('num', 1))), ('ret', ('name', 'q'))]


@pytest.mark.parametrize('bad', ['a[i] = ', 'x = (1 + 2', 'z[n] = fold step i: w\n', 'q = 1 2'])
def test_syntax_errors_name_the_line(bad):
    with pytest.raises(SyntaxError, match='line'):
        fe.parse(bad + '\n' if 'fold step' not in bad else bad + 'end\n')


def test_missing_end():
    with pytest.raises(SyntaxError, match='missing end'):
        fe.parse('z[n] = fold step i: w as c\n  -> c\n')


@pytest.mark.parametrize('name', ['gpt2.vst', 'gpt2_medium.vst', 'gpt2_xl.vst'])
def test_programs_parse_same_in_both_parsers(name):
    text = open(os.path.join(PROGRAMS, name)).read()
    assert fe.parse(text) == oracle.parse(text)


def test_committed_programs_are_the_template():
    assert open(os.path.join(PROGRAMS, 'gpt2.vst')).read() == gpt2_program(12, 768, 12, 3072, 50257, 'small')
    assert open(os.path.join(PROGRAMS, 'gpt2_medium.vst')).read() == gpt2_program(24, 1024, 16, 4096, 50257, 'medium')
    assert open(os.path.join(PROGRAMS, 'gpt2_xl.vst')).read() == gpt2_program(48, 1600, 25, 6400, 50257, 'XL')


@pytest.mark.skipif(not os.path.exists(os.path.join(REFERENCE, 'vesta/programs/gpt2.vst')), reason='reference tree absent')
def test_reference_program_text_parses_to_same_ast():
    ref = open(os.path.join(REFERENCE, 'vesta/programs/gpt2.vst')).read()
    mine = open(os.path.join(PROGRAMS, 'gpt2.vst')).read()
    assert fe.parse(ref) == fe.parse(mine)
