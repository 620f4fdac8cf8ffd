"""The oracle's serial orders, pinned by inputs that separate them.

Each test restates one of Trit's sequences from its Rust source with exact
arithmetic (every product and sum held as a rational, then rounded once to
the nearest float32, ties to even -- a fused multiply-add exactly), searches
inputs on which the plausible misreadings (another order, a tree, a fused
step left unfused or the reverse) give other bits, and checks the oracle
against the restatement on them:

- the exp steps of the fused paths (src/cpu/activation.rs:357-375);
- RMSNorm's sum of squares, one after another from 0 (src/layers.rs:136-144);
- attention's score chain over the dims, softmax sum over the keys and p.V
  chain over the keys (src/layers.rs:442-504,571-587; the fused tiles of
  src/cpu/fgemm.rs:665-793; add_columns, src/cpu/activation.rs:133-152).
"""

from fractions import Fraction as F

import numpy as np

from oracle import oracle as O

f32 = np.float32


def round32(x: F) -> np.float32:
    """The float32 nearest the rational x, ties to the even significand."""
    if x == 0:
        return f32(0.0)
    r = f32(float(x))  # float(x) is x rounded to binary64; r is then within one step of the answer
    if F(float(r)) == x:
        return r
    cands = [np.nextafter(r, f32(-np.inf)), r, np.nextafter(r, f32(np.inf))]
    return min(cands, key=lambda c: (abs(F(float(c)) - x), int(f32(c).view(np.uint32)) & 1))


def fma(a, b, c) -> np.float32:
    return round32(F(float(a)) * F(float(b)) + F(float(c)))


def bits(v):
    return np.asarray(v, np.float32).view(np.uint32)


# ---- exp (activation.rs:8-45 constants, :357-375 the fused steps) ---------

LOG2E, LN2_HI, LN2_LO = f32(1.4426950408889634), f32(0.6933594), f32(-2.1219444e-4)
LOW, HIGH = f32(-87.3), f32(88.0)
POLY = [f32(v) for v in (1.9875691e-4, 1.3981999e-3, 8.333452e-3, 4.1665796e-2, 0.16666665, 0.5)]


def exp_fused(x: np.float32) -> np.float32:
    """x clamped; n = round-to-even(x log2 e); r = x - n ln2_hi - n ln2_lo,
    each a fused step; p by fused Horner steps from 0; y = p (r r) + (r + 1)
    fused; y 2^n."""
    x = min(max(f32(x), LOW), HIGH)
    n_int = int(np.rint(f32(x * LOG2E)))
    n = f32(n_int)
    r = fma(-n, LN2_HI, x)
    r = fma(-n, LN2_LO, r)
    p = f32(0.0)
    for c in POLY:
        p = fma(p, r, c)
    y = fma(p, f32(r * r), f32(r + f32(1.0)))
    return f32(y * f32(2.0 ** n_int))


def exp_unfused(x: np.float32) -> np.float32:
    """The scalar path's steps (activation.rs:186-193): every product and sum
    rounded on its own."""
    x = min(max(f32(x), LOW), HIGH)
    n = f32(np.rint(f32(x * LOG2E)))
    r = f32(f32(x - f32(n * LN2_HI)) - f32(n * LN2_LO))
    p = f32(0.0)
    for c in POLY:
        p = f32(f32(p * r) + c)
    return f32(f32(f32(f32(p * r) * r) + r) + f32(1.0)) * f32(2.0 ** int(n))


def test_exp_fused_steps():
    rng = np.random.default_rng(11)
    xs = np.concatenate([rng.uniform(-90, 90, 1500), rng.uniform(-1, 1, 600), rng.normal(0, 1e-3, 200),
                         [0.0, -0.0, 1.0, -1.0, 88.0, 88.5, -87.3, -100.0, 0.5, -0.5, 1e-30]]).astype(np.float32)
    want = np.array([exp_fused(x) for x in xs], np.float32)
    got = np.array([O.exp(float(x)) for x in xs], np.float32)
    assert np.array_equal(bits(got), bits(want)), xs[bits(got) != bits(want)][:5]
    # The unfused steps are another function: the test tells them apart.
    other = np.array([exp_unfused(x) for x in xs], np.float32)
    assert np.count_nonzero(bits(other) != bits(want)) > 50


# ---- RMSNorm (layers.rs:136-144) -------------------------------------------

def rmsnorm_row(x, w, eps):
    """sum = ((0 + x0 x0) + x1 x1) + ..., each square rounded; inv =
    1 / sqrt(sum / d + eps); x * (inv * w)."""
    s = f32(0.0)
    for v in x:
        s = f32(s + f32(v * v))
    inv = f32(f32(1.0) / np.sqrt(f32(f32(s / f32(len(x))) + f32(eps))))
    return np.array([f32(v * f32(inv * wi)) for v, wi in zip(x, w)], np.float32)


def finish(s, x, w, eps):
    inv = f32(f32(1.0) / np.sqrt(f32(f32(s / f32(len(x))) + f32(eps))))
    return np.array([f32(v * f32(inv * wi)) for v, wi in zip(x, w)], np.float32)


def test_rmsnorm_sum_order():
    """Rows whose outputs change under a tree sum, the reverse order or a
    fused square-and-add, against the oracle on every row."""
    rng = np.random.default_rng(13)
    d, eps, found = 64, 1e-6, 0
    w = (1 + 0.25 * rng.standard_normal(d)).astype(np.float32)
    for _ in range(400):
        x = (rng.standard_normal(d) * np.exp(rng.uniform(-3, 3, d))).astype(np.float32)
        want = rmsnorm_row(x, w, eps)
        got = O.rmsnorm(x.reshape(1, d), w, eps)[0]
        assert np.array_equal(bits(got), bits(want))
        sq = [f32(v * v) for v in x]
        tree = sq
        while len(tree) > 1:
            tree = [f32(tree[i] + tree[i + 1]) for i in range(0, len(tree), 2)]
        rev = f32(0.0)
        for q in reversed(sq):
            rev = f32(rev + q)
        fused = f32(0.0)
        for v in x:
            fused = fma(v, v, fused)
        alts = [finish(s, x, w, eps) for s in (tree[0], rev, fused)]
        if all(not np.array_equal(bits(a), bits(want)) for a in alts):
            found += 1
    assert found >= 10  # rows that tell the orders apart were among those checked (18 with this seed)


# ---- attention (layers.rs:442-504,571-587) ----------------------------------

def attention_row(q, k, v):
    """One query over tk keys of one head: qh = q (1/sqrt(hd)); s_j = fused
    chain of qh_e k_je over e from 0; m = max; e_j = exp(s_j - m); sum =
    ((0 + e_0) + e_1) + ...; p_j = e_j (1 / sum); out_e = fused chain of
    p_j v_je over j from 0."""
    hd = q.size
    scale = f32(f32(1.0) / np.sqrt(f32(hd)))
    qh = [f32(x * scale) for x in q]
    s = []
    for kr in k:
        acc = f32(0.0)
        for e in range(hd):
            acc = fma(qh[e], kr[e], acc)
        s.append(acc)
    m = max(s)
    ex = [exp_fused(f32(sj - m)) for sj in s]
    tot = f32(0.0)
    for x in ex:
        tot = f32(tot + x)
    inv = f32(f32(1.0) / tot)
    p = [f32(x * inv) for x in ex]
    out = []
    for e in range(hd):
        acc = f32(0.0)
        for j in range(len(p)):
            acc = fma(p[j], v[j][e], acc)
        out.append(acc)
    return np.array(out, np.float32), s, ex, p


def test_attention_orders():
    """The score chain, the softmax sum and the p.V chain each in key / dim
    order from 0: the oracle equals the restatement on every case, and each
    misreading (dims reversed or unfused in the scores, a tree softmax sum,
    keys reversed or unfused in p.V) changes the output of some case."""
    rng = np.random.default_rng(17)
    hd, tk = 8, 12
    seen = {"scores": 0, "sum": 0, "pv": 0}
    for trial in range(40):
        q = (rng.standard_normal(hd) * 3).astype(np.float32)
        k = (rng.standard_normal((tk, hd)) * np.exp(rng.uniform(-1, 1, (tk, 1)))).astype(np.float32)
        v = (rng.standard_normal((tk, hd)) * np.exp(rng.uniform(-2, 2, (tk, hd)))).astype(np.float32)
        want, s, ex, p = attention_row(q, k, v)
        got = O.attention(q.reshape(1, hd), k, v, 1, 1, hd, causal=False)[0]
        assert np.array_equal(bits(got), bits(want)), trial
        # Scores: dims in reverse, or each product rounded before the add.
        scale = f32(f32(1.0) / np.sqrt(f32(hd)))
        qh = [f32(x * scale) for x in q]
        for kr, sj in zip(k, s):
            r = f32(0.0)
            for e in reversed(range(hd)):
                r = fma(qh[e], kr[e], r)
            u = f32(0.0)
            for e in range(hd):
                u = f32(u + f32(qh[e] * kr[e]))
            if r != sj and u != sj:
                seen["scores"] += 1
                break
        # The softmax sum as a pairwise tree.
        tree = list(ex) + [f32(0.0)] * (16 - tk)
        while len(tree) > 1:
            tree = [f32(tree[i] + tree[i + 1]) for i in range(0, len(tree), 2)]
        tot = f32(0.0)
        for x in ex:
            tot = f32(tot + x)
        if tree[0] != tot:
            seen["sum"] += 1
        # p.V: keys reversed, or unfused.
        for e in range(hd):
            r = f32(0.0)
            for j in reversed(range(tk)):
                r = fma(p[j], v[j][e], r)
            u = f32(0.0)
            for j in range(tk):
                u = f32(u + f32(p[j] * v[j][e]))
            if r != want[e] and u != want[e]:
                seen["pv"] += 1
                break
    assert all(n >= 5 for n in seen.values()), seen
