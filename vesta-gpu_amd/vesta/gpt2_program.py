"""GPT-2 decode-step program text for any GPT-2 extents.

The committed programs ``programs/gpt2.vst`` (small), ``gpt2_medium.vst`` and
``gpt2_xl.vst`` are this text at those extents; tests also use it at tiny
extents. The statements, residue names and shapes are those the decode API
binds by name (reference ``vesta/programs/gpt2.vst:3-82``, ``vesta/gpt2.py:21-25``).
"""
import math

TEMPLATE = '''# GPT-2 {label}: one greedy decode step for one token.
# Q1..Q10 name the questions a decode step answers (embed, layer norm, qkv,
# cache, scores, softmax, attention output, mlp, logits, argmax).

residue x                        # token id
residue t                        # its position

axis d = {d}
axis h = {h}
axis e = {e}
axis f = {f}
axis n = {n}
axis j = {j}
axis l = {L}
axis s = t + 1                   # positions 0..t

residue wte[n, d]
residue wpe[s, d]
residue ln1w[l, d]
residue ln1b[l, d]
residue qkvw[l, d, j]
residue qkvb[l, j]
residue ow[l, d, d]
residue ob[l, d]
residue ln2w[l, d]
residue ln2b[l, d]
residue fcw[l, d, f]
residue fcb[l, f]
residue pw[l, f, d]
residue pb[l, d]
residue lnfw[d]
residue lnfb[d]
residue keys[l, s, h, e]
residue vals[l, s, h, e]

# Q1  token meaning plus position meaning
z0[d] = wte[x, d] + wpe[t, d]

zL[d] = fold step l: z0 as z
    # Q2  normalise (biased variance, eps 1e-5)
    m1 = fold sum d: z[d] / {d}
    v1 = fold sum d: (z[d] - m1) * (z[d] - m1) / {d}
    a[d] = (z[d] - m1) / sqrt(v1 + 0.00001) * ln1w[l, d] + ln1b[l, d]

    # Q3  query, key, value
    qkv[j] = (fold sum d: a[d] * qkvw[l, d, j]) + qkvb[l, j]
    q[h, e] = qkv[h * {e} + e]

    # Q4  this position's key and value join the cache
    residue keys[l, t, h, e] <- qkv[{d} + h * {e} + e]
    residue vals[l, t, h, e] <- qkv[{d2} + h * {e} + e]

    # Q5  scores, scaled by 1/sqrt({e})
    sc[h, s] = (fold sum e: q[h, e] * keys[l, s, h, e]) / {rs}

    # Q6  softmax over positions
    mx[h] = fold max s: sc[h, s]
    ex[h, s] = exp(sc[h, s] - mx[h])
    w[h, s] = ex[h, s] / (fold sum s: ex[h, s])

    # Q7  weighted values, joined heads, projection, residual
    o[h, e] = fold sum s: w[h, s] * vals[l, s, h, e]
    oo[d] = fold sum h: (fold sum e: o[h, e] * ow[l, h * {e} + e, d])
    z1[d] = z[d] + oo[d] + ob[l, d]

    # Q8  normalise, widen with tanh-GELU, narrow, residual
    m2 = fold sum d: z1[d] / {d}
    v2 = fold sum d: (z1[d] - m2) * (z1[d] - m2) / {d}
    b[d] = (z1[d] - m2) / sqrt(v2 + 0.00001) * ln2w[l, d] + ln2b[l, d]
    u[f] = (fold sum d: b[d] * fcw[l, d, f]) + fcb[l, f]
    g[f] = 0.5 * u[f] * (1 + tanh(0.7978845608028654 * (u[f] + 0.044715 * u[f] * u[f] * u[f])))
    z2[d] = z1[d] + (fold sum f: g[f] * pw[l, f, d]) + pb[l, d]
    -> z2
end

# Q9  final norm, then the tied word table as the output head
m3 = fold sum d: zL[d] / {d}
v3 = fold sum d: (zL[d] - m3) * (zL[d] - m3) / {d}
c[d] = (zL[d] - m3) / sqrt(v3 + 0.00001) * lnfw[d] + lnfb[d]
logit[n] = fold sum d: c[d] * wte[n, d]

# Q10 the highest score; a tie goes to the lowest id
best = fold max n: logit[n]
next = fold min n: fork logit[n] == best ? n : {n}
'''


def gpt2_program(n_layer: int, d: int, n_head: int, f: int, vocab: int = 50257, label: str = 'custom') -> str:
    """Program text at these extents. The head width must be a perfect square
    (the score scale 1/sqrt(head width) is written as an integer divisor)."""
    e = d // n_head
    rs = math.isqrt(e)
    if e * n_head != d or rs * rs != e:
        raise ValueError(f'head width {e} must divide d and be a perfect square')
    return TEMPLATE.format(label=label, L=n_layer, d=d, h=n_head, e=e, f=f, n=vocab, j=3 * d, d2=2 * d, rs=rs)
