"""trit_hip_attention (layers::attention, src/layers.rs:343-504) against the
oracle: the exact form bit for bit, the fast form (f16 keys and values, the
matrix cores) within 1e-3 of the oracle run on the same f16-rounded keys and
values.

Output row i of causal attention depends only on query row i and the keys
and values it sees, and masked keys add exact zeros to the oracle's sums,
so the oracle is run row by row on a sample of rows (query tile edges and
the longest rows included) with exactly the keys each sees.
"""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, synth

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def inputs(seed, tq, tk, heads, kv_heads, hd):
    q = synth.normal(synth.seed_for(seed, 1), (tq, heads * hd)).astype(np.float32)
    k = synth.normal(synth.seed_for(seed, 2), (tk, kv_heads * hd)).astype(np.float32)
    v = synth.normal(synth.seed_for(seed, 3), (tk, kv_heads * hd)).astype(np.float32)
    return q, k, v


def oracle_rows(q, k, v, rows, heads, kv_heads, hd, causal):
    tq, tk = q.shape[0], k.shape[0]
    out = []
    for i in rows:
        seen = tk - tq + i + 1 if causal else tk
        out.append(O.attention(q[i:i + 1], k[:seen], v[:seen], heads, kv_heads, hd, causal=False)[0])
    return np.array(out)


def sample_rows(tq, seed):
    edges = [0, 1, 15, 16, 31, 32, 63, 64, tq // 2, tq - 33, tq - 32, tq - 2, tq - 1]
    return sorted(set(r for r in edges + synth.ints(seed, (12,), 0, tq - 1).tolist() if 0 <= r < tq))


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("tq,tk,heads,kv_heads,causal", [
    (1564, 1564, 16, 8, True),   # the prefill configuration's attention
    (100, 700, 16, 8, True),     # a continuation: queries at positions 600..699
    (300, 300, 8, 8, True),
    (250, 250, 16, 4, False),    # without a mask (an encoder's attention)
])
def test_attention(gpu, tq, tk, heads, kv_heads, causal):
    print(f"case attention tq={tq} tk={tk} heads={heads}/{kv_heads} causal={causal}", flush=True)
    hd = 128
    q, k, v = inputs(60 + tq, tq, tk, heads, kv_heads, hd)
    rows = sample_rows(tq, 61 + tq)
    exact = hip.attention(q, k, v, heads, kv_heads, hd, causal, hip.EXACT)
    want = oracle_rows(q, k, v, rows, heads, kv_heads, hd, causal)
    assert bits_equal(exact[rows], want), rel(exact[rows], want)
    fast = hip.attention(q, k, v, heads, kv_heads, hd, causal, 0)
    assert np.all(np.isfinite(fast))
    k16 = k.astype(np.float16).astype(np.float32)
    v16 = v.astype(np.float16).astype(np.float32)
    want16 = oracle_rows(q, k16, v16, rows, heads, kv_heads, hd, causal)
    print(f"fast vs the oracle on f16 keys and values {rel(fast[rows], want16):.3g}", flush=True)
    assert rel(fast[rows], want16) < 1e-3
    # Every row of the fast form against the exact form (f32 keys and values):
    # within what f16 keys and values move a row.
    assert rel(fast, exact) < 2e-2


def test_attention_masked_tail_exact(gpu):
    """Keys past a causal block's last row weigh exp_trit(-inf) / sum (about
    1e-38): the exact kernel leaves them out only where they cannot move a
    chain. Here every key a row sees has value 0 and the later keys 1000,
    so the rows' outputs are those tiny masked terms alone, and they must
    match Trit's attention over every key, bit for bit."""
    print("case attention exact masked tail", flush=True)
    tq = tk = 70
    heads, hd = 2, 64
    q, k, v = inputs(67, tq, tk, heads, heads, hd)
    v[:60] = 0.0
    v[60:] = 1000.0
    got = hip.attention(q, k, v, heads, heads, hd, True, hip.EXACT)
    want = O.attention(q, k, v, heads, heads, hd, causal=True)
    assert bits_equal(got, want)
    assert np.any(got[:56] != 0.0)  # the masked terms reached the outputs


def test_attention_small_heads_exact(gpu):
    """The exact form at head_dim 64 (Whisper-size heads), no mask."""
    print("case attention exact hd 64", flush=True)
    q, k, v = inputs(66, 40, 90, 6, 6, 64)
    got = hip.attention(q, k, v, 6, 6, 64, False, hip.EXACT)
    want = O.attention(q, k, v, 6, 6, 64, causal=False)
    assert bits_equal(got, want)


def test_attention_errors(gpu):
    q, k, v = inputs(67, 4, 8, 2, 2, 64)
    with pytest.raises(hip.TritError, match="fast form"):
        hip.attention(q, k, v, 2, 2, 64, True, 0)
    with pytest.raises(hip.TritError, match="more queries"):
        hip.attention(np.zeros((9, 128), np.float32), k, v, 2, 2, 64, True, hip.EXACT)
