"""Whisper's audio encoder on the device (trit_hip_encoder_encode) against
the oracle's Encoder, bit for bit: the stem's im2col and convolutions, the
exact GELU, layer norm in Trit's 32-lane order, the attention with no mask,
the MLP and residual adds -- with Q8_0 products (int8 activations, the
matrix cores where the shape allows) and an f16 first convolution (80 mel
bins: 240 inputs, f32 math)."""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, synth

pytestmark = pytest.mark.gpu


def make(cfg, seed, conv1_f16=False):
    """Device layers and the oracle's products for the same weights."""
    d, ffn, mels, P = cfg["d"], cfg["ffn"], cfg["mels"], cfg["positions"]
    t = [0]
    isa = O.isa_best()

    def nxt():
        t[0] += 1
        return synth.seed_for(seed, t[0])

    def vec(n, base=0.0, spread=0.2):
        return (base + spread * (2 * synth.uniform(nxt(), n) - 1)).astype(np.float32)

    def q8(n, k, zero_from=None):
        codes, sbits = synth.q8_0_matrix(nxt(), n, k, scale="normal", sigma=0.2)
        bias = vec(n)
        if zero_from is not None:
            bias[zero_from[0]:zero_from[1]] = 0.0  # the stacked k's missing bias
        dev = hip.Dense.q8_0(n, k, synth.q8_0_blocks(codes, sbits), bias)
        lay = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True, isa)
        return dev, (lambda x, lay=lay, b=bias: (lay(np.ascontiguousarray(x, np.float32)) + b).astype(np.float32))

    def f16(n, k):
        w = synth.f16_bits((synth.normal(nxt(), (n, k)) / np.sqrt(k)).astype(np.float32))
        bias = vec(n)
        dev = hip.Dense.f16(w, bias)
        return dev, (lambda x, w=w, b=bias: (O.matmul_f16(np.ascontiguousarray(x, np.float32), w, isa) + b)
                     .astype(np.float32))

    conv1 = f16(d, 3 * mels) if conv1_f16 else q8(d, 3 * mels)
    conv2 = q8(d, 3 * d)
    devs, prods, norms = [], [conv1[1], conv2[1]], []
    for _ in range(cfg["layers"]):
        for dev, prod in (q8(3 * d, d, (d, 2 * d)), q8(d, d), q8(ffn, d), q8(d, ffn)):
            devs.append(dev)
            prods.append(prod)
        norms += [vec(d, 1.0), vec(d), vec(d, 1.0), vec(d)]
    norms += [vec(d, 1.0), vec(d)]
    positions = vec(P * d, 0.0, 0.5).reshape(P, d)
    enc = hip.Encoder(cfg, conv1[0], conv2[0], positions, devs, norms)
    ref = O.Encoder(cfg, prods, positions, norms)
    return enc, ref


@pytest.mark.parametrize("cfg,conv1_f16", [
    (dict(d=128, layers=2, heads=4, ffn=256, mels=32, positions=24), False),
    (dict(d=512, layers=2, heads=8, ffn=2048, mels=80, positions=1500), True),  # Whisper base's shapes, 2 layers
])
def test_encoder_against_oracle(gpu, cfg, conv1_f16):
    print(f"case audio encoder {cfg}", flush=True)
    enc, ref = make(cfg, 150 + cfg["d"], conv1_f16)
    mel = synth.activations(151, 2 * cfg["positions"], cfg["mels"])
    got = enc.encode(mel)
    want = ref.encode(mel)
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    print(f"  max rel diff {err:.3g}", flush=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
