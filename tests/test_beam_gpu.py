"""A decoder step with several sequences (beam search, Whisper's 5 beams):
layers::attention_steps (src/layers.rs:505-562) and the f16 products of 5
rows with bias, against the oracle, bit for bit."""

import numpy as np
import pytest

from oracle import oracle as O
from tests.device_memory import Device
from trit_amd import hip, synth

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def caches(seed, tks, kvs):
    return [(synth.activations(seed + 2 * i, tk, kvs), synth.activations(seed + 2 * i + 1, tk, kvs))
            for i, tk in enumerate(tks)]


# (d, heads, kv_heads, key counts per sequence, query stride)
SHAPES = [
    (1280, 20, 20, [1, 17, 64, 200, 448], 1280),  # Whisper large-v3's decoder, 5 beams
    (384, 6, 6, [3, 5, 9, 2, 448], 3 * 384),  # Whisper tiny, queries inside qkv rows
    (2048, 16, 8, [300, 1, 1000, 33], 2048 + 2 * 1024),  # grouped heads (Qwen3-0.6B's)
    (512, 4, 1, [7], 512),  # one sequence, one key head
]


@pytest.mark.parametrize("d,heads,kv_heads,tks,qs", SHAPES)
def test_attention_steps(gpu, d, heads, kv_heads, tks, qs):
    print(f"case attention_steps d={d} heads={heads}/{kv_heads} tk={tks}", flush=True)
    hd = d // heads
    q = synth.activations(700 + d, len(tks), qs)
    cs = caches(710 + d, tks, kv_heads * hd)
    want = O.attention_steps(q, cs, heads, kv_heads)
    got = hip.attention_steps(q, cs, heads, kv_heads)
    assert bits_equal(got, want)
    # Each row is the exact attention of that sequence alone.
    for b, (k, v) in enumerate(cs):
        one = hip.attention(q[b:b + 1, :d], k, v, heads, kv_heads, hd, causal=False, flags=hip.EXACT)
        assert bits_equal(got[b], one[0])


def test_attention_steps_device(gpu):
    """The device-memory entry point: the same bits, queued on the calling
    thread's stream."""
    import ctypes as C

    print("case attention_steps on device memory", flush=True)
    d, heads, kv_heads, tks, qs = SHAPES[0]
    hd = d // heads
    q = synth.activations(720, len(tks), qs)
    cs = caches(730, tks, kv_heads * hd)
    want = hip.attention_steps(q, cs, heads, kv_heads)
    D = Device()
    try:
        dq = D.upload(q)
        keys = (C.c_void_p * len(tks))(*[D.upload(k).value for k, _ in cs])
        values = (C.c_void_p * len(tks))(*[D.upload(v).value for _, v in cs])
        tk = (C.c_int * len(tks))(*tks)
        dout = D.empty(len(tks) * d * 4)
        hip.check(hip.lib().trit_hip_attention_steps_device(dq, qs, keys, values, tk, len(tks), d, heads, kv_heads,
                                                            dout, None))
        got = D.download(dout, (len(tks), d))
    finally:
        D.free()
    assert bits_equal(got, want)


def test_attention_steps_errors(gpu):
    print("case attention_steps errors", flush=True)
    q = np.zeros((2, 256), np.float32)
    k = np.zeros((4, 256), np.float32)
    with pytest.raises(hip.TritError, match="no keys"):
        hip.attention_steps(q, [(k, k), (k[:0], k[:0])], 4, 4)
    with pytest.raises(hip.TritError, match="1 to 32"):
        hip.attention_steps(np.zeros((33, 256), np.float32), [(k, k)] * 33, 4, 4)
    with pytest.raises(hip.TritError, match="share"):
        hip.attention_steps(q, [(k, k), (k, k)], 4, 3)


@pytest.mark.parametrize("n,k", [(1280, 1280), (5120, 1280), (1280, 5120), (51866, 1280)])
def test_beam_products(gpu, n, k):
    """The f16 products of a Whisper large-v3 decoder step with 5 beams
    (q/k/v/o 1280x1280, fc1 5120x1280, fc2 1280x5120, the tied token
    table's 51866x1280), with bias where Whisper has one."""
    print(f"case beam f16 product n={n} k={k} rows=5", flush=True)
    w = synth.f16_bits(synth.activations(740 + n, n, k) * 0.02).reshape(n, k)
    bias = None if n == 51866 else synth.activations(741 + n, 1, n)[0]
    x = synth.activations(742 + k, 5, k)
    want = O.matmul_f16(x, w)
    if bias is not None:
        want = want + bias
    got = hip.Dense.f16(w, bias).forward(x)
    assert bits_equal(got, want)
