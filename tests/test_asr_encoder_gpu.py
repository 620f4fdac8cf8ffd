"""The Qwen3-ASR audio encoder on the device (trit_hip_asr_encoder_encode)
against the oracle's AsrEncoder, bit for bit: the chunk maps zero padded to
the longest chunk, three 3x3 stride-2 convolutions with the exact GELU, the
channel-major time columns, conv_out, the sinusoid positions, attention
within windows, the MLPs, ln_post and the projections -- with Q8_0
products (int8 activations; the matrix cores for many rows, K tails
included: 9 * 480 = 4320 inputs), f32 math for the 9-input first
convolution, and f16 / f32 layers where the shapes are not Q8_0's."""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, synth

pytestmark = pytest.mark.gpu


def make(cfg, seed, small):
    """Device layers and the oracle's products for the same weights. small:
    the convolutions after the first, conv_out and proj2 as f16 / f32
    layers (their shapes are not Q8_0's)."""
    d, ffn, ch, out = cfg["d"], cfg["ffn"], cfg["channels"], cfg["out"]
    bins = cfg["mels"]
    for _ in range(3):
        bins = (bins + 1) // 2
    t = [0]
    isa = O.isa_best()

    def nxt():
        t[0] += 1
        return synth.seed_for(seed, t[0])

    def vec(n, base=0.0, spread=0.2):
        return (base + spread * (2 * synth.uniform(nxt(), n) - 1)).astype(np.float32)

    def q8(n, k):
        codes, sbits = synth.q8_0_matrix(nxt(), n, k, scale="normal", sigma=0.2)
        bias = vec(n)
        dev = hip.Dense.q8_0(n, k, synth.q8_0_blocks(codes, sbits), bias)
        lay = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True, isa)
        return dev, (lambda x, lay=lay, b=bias: (lay(np.ascontiguousarray(x, np.float32)) + b).astype(np.float32))

    def f16(n, k):
        w = synth.f16_bits((synth.normal(nxt(), (n, k)) / np.sqrt(k)).astype(np.float32))
        bias = vec(n)
        return hip.Dense.f16(w, bias), (lambda x, w=w, b=bias: (O.matmul_f16(np.ascontiguousarray(x, np.float32), w,
                                                                                isa) + b).astype(np.float32))

    def f32(n, k):
        w = (synth.normal(nxt(), (n, k)) / np.sqrt(k)).astype(np.float32)
        bias = vec(n)
        return hip.Dense.f32(w, bias), (lambda x, w=w, b=bias: (O.matmul_f32(np.ascontiguousarray(x, np.float32), w,
                                                                                isa) + b).astype(np.float32))

    convs = [f32(ch, 9)] + [(f16 if small else q8)(ch, 9 * ch) for _ in range(2)]
    conv_out = (f32 if small else q8)(d, ch * bins)
    devs, prods, norms = [], [c[1] for c in convs] + [conv_out[1]], []
    for _ in range(cfg["layers"]):
        for dev, prod in (q8(3 * d, d), q8(d, d), q8(ffn, d), q8(d, ffn)):
            devs.append(dev)
            prods.append(prod)
        norms += [vec(d, 1.0), vec(d), vec(d, 1.0), vec(d)]
    norms += [vec(d, 1.0), vec(d)]
    proj1, proj2 = q8(d, d), (f16 if small else q8)(out, d)
    prods += [proj1[1], proj2[1]]
    enc = hip.AsrEncoder(cfg, [c[0] for c in convs], conv_out[0], devs, norms, proj1[0], proj2[0])
    ref = O.AsrEncoder(cfg, prods, norms)
    return enc, ref


SMALL = dict(d=64, layers=2, heads=4, ffn=128, mels=16, channels=8, chunk=32, window_chunks=2, out=48,
             max_positions=40)
# Qwen3-ASR's stem (128 mel bins, 480 channels, chunks of 100 frames,
# windows of 8 chunks) under a 512-wide, 2-layer stack.
STEM = dict(d=512, layers=2, heads=8, ffn=2048, mels=128, channels=480, chunk=100, window_chunks=8, out=1024,
            max_positions=1500)


@pytest.mark.parametrize("cfg,frames,small", [(SMALL, 108, True), (SMALL, 32, True), (SMALL, 7, True),
                                              (SMALL, 300, True), (STEM, 1037, False)])
def test_asr_encoder_against_oracle(gpu, cfg, frames, small):
    print(f"case asr encoder d={cfg['d']} channels={cfg['channels']} frames={frames}", flush=True)
    enc, ref = make(cfg, 170 + cfg["d"] + frames, small)
    assert np.array_equal(enc.positions().view(np.uint32), ref.positions.view(np.uint32))
    assert enc.rows(frames) == ref.rows(frames)
    mel = synth.activations(171 + frames, frames, cfg["mels"])
    got = enc.encode(mel, frames)
    want = ref.encode(mel, frames)
    assert got.shape == want.shape
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    print(f"  rows {got.shape[0]}, max rel diff {err:.3g}", flush=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_asr_encoder_refusals(gpu):
    print("case asr encoder refusals", flush=True)
    enc, _ = make(SMALL, 5, True)
    with pytest.raises(hip.TritError):
        enc.encode(np.zeros((0, SMALL["mels"]), np.float32), 0)
    bad = dict(SMALL, max_positions=1)
    with pytest.raises(hip.TritError, match="max_positions"):
        make(bad, 6, True)
