"""The oracle's audio encoder (Encoder::encode, src/models/parts/
audio_encoder.rs:111-138) pinned: its pieces against the mathematics (the
exact GELU against erf, layer norm against float64, im2col against direct
indexing) and its composition against a float64 Whisper encoder written
from the model definition, with planted mistakes that the check catches."""

import numpy as np
import pytest
from scipy.special import erf

from oracle import oracle as O
from tests import whisper_float64 as W
from trit_amd import synth

ENC = dict(d=128, layers=2, heads=4, ffn=256, mels=32, positions=24)
TOL = 2e-5  # of the largest output: f32 against float64
MISTAKE_TOL = 10 * TOL  # a planted mistake moves the output at least this far
MISTAKES = ["tanh_gelu", "conv2_shift", "post_norm", "positions_before_gelu", "causal"]


def test_gelu_against_erf():
    x = np.concatenate([np.linspace(-12, 12, 20001), [0.0, -0.0, 1e-30, -1e-30, 1e-3, -1e-3]]).astype(np.float32)
    got = O.gelu(x).astype(np.float64)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1 + erf(xd / np.sqrt(2)))
    # Numerical Recipes' erfc is within 1.2e-7 relative; exp within ~2 ulp.
    assert np.all(np.abs(got - want) <= 2e-6 * np.abs(xd) + 1e-12)
    assert O.gelu(np.float32([0.0]))[0] == 0.0
    assert np.array_equal(O.gelu(np.float32([9.0, 20.0])), np.float32([9.0, 20.0]))


def test_layer_norm_against_float64():
    x = synth.activations(300, 7, 200) * np.float32(3) + np.float32(1.5)
    w = synth.activations(301, 1, 200)[0]
    b = synth.activations(302, 1, 200)[0]
    got = O.layer_norm(x, w, b)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(got - want)) < 1e-5 * np.max(np.abs(want))
    # The sums' order: 32 lanes (lane j: values j, j + 32, ...), added in
    # order, then the tail. Lane 0 holds 1e8 and 1 (1 is lost: 1e8 + 1 ==
    # 1e8 in f32), lane 1 holds -1e8: the mean is exactly 0, so a zero
    # value stays exactly 0. One chain in row order would keep the 1 (mean
    # 1/64) and move the zero.
    row = np.zeros((1, 64), np.float32)
    row[0, 0], row[0, 32], row[0, 1] = 1e8, 1.0, -1e8
    out = O.layer_norm(row, np.ones(64, np.float32), np.zeros(64, np.float32))
    assert out[0, 2] == 0.0
    chain = np.float32(0)
    for v in row[0]:
        chain = np.float32(chain + v)
    assert chain != 0  # the other order would not give 0


def test_conv_columns_direct():
    x = synth.activations(310, 11, 5)
    for kernel, stride, pad, out_frames in [(3, 1, 1, 11), (3, 2, 1, 6), (5, 1, 2, 11)]:
        got = O.conv_columns(x, kernel, stride, pad, out_frames)
        for t in range(out_frames):
            for tap in range(kernel):
                src = t * stride + tap - pad
                col = x[src] if 0 <= src < 11 else np.zeros(5, np.float32)
                assert np.array_equal(got[t, tap::kernel], col)


def make(cfg, seed):
    """Random f32 weights for both sides: the oracle's f32 products (with
    bias) and the float64 model."""
    d, ffn, mels, P = cfg["d"], cfg["ffn"], cfg["mels"], cfg["positions"]
    t = [0]

    def mat(*shape):
        t[0] += 1
        fan = int(np.prod(shape[1:]))
        return (synth.normal(synth.seed_for(seed, t[0]), shape) / np.sqrt(fan)).astype(np.float32)

    def vec(n, base=0.0, spread=0.2):
        t[0] += 1
        return (base + spread * (2 * synth.uniform(synth.seed_for(seed, t[0]), n) - 1)).astype(np.float32)

    p = dict(conv1_w=mat(d, mels, 3), conv1_b=vec(d), conv2_w=mat(d, d, 3), conv2_b=vec(d),
             positions=vec(P * d, 0.0, 0.5).reshape(P, d), norm_w=vec(d, 1.0), norm_b=vec(d), layers=[])
    for _ in range(cfg["layers"]):
        p["layers"].append(dict(q=mat(d, d), k=mat(d, d), v=mat(d, d), o=mat(d, d), fc1=mat(ffn, d),
                                fc2=mat(d, ffn), bq=vec(d), bv=vec(d), bo=vec(d), b1=vec(ffn), b2=vec(d),
                                attn_w=vec(d, 1.0), attn_b=vec(d), ffn_w=vec(d, 1.0), ffn_b=vec(d)))
    return p


def oracle_encoder(cfg, p):
    """O.Encoder with f32 products: conv weights as [out][in * 3] (the
    [out][in][kernel] order im2col's columns follow)."""
    d = cfg["d"]

    def f32(w, b):
        w = np.ascontiguousarray(w.reshape(w.shape[0], -1), np.float32)
        return lambda x: (O.matmul_f32(np.ascontiguousarray(x, np.float32), w) + b).astype(np.float32)

    products = [f32(p["conv1_w"], p["conv1_b"]), f32(p["conv2_w"], p["conv2_b"])]
    norms = []
    for L in p["layers"]:
        qkv = np.concatenate([L["q"], L["k"], L["v"]])
        bqkv = np.concatenate([L["bq"], np.zeros(d, np.float32), L["bv"]])
        products += [f32(qkv, bqkv), f32(L["o"], L["bo"]), f32(L["fc1"], L["b1"]), f32(L["fc2"], L["b2"])]
        norms += [L["attn_w"], L["attn_b"], L["ffn_w"], L["ffn_b"]]
    norms += [p["norm_w"], p["norm_b"]]
    return O.Encoder(cfg, products, p["positions"], norms)


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def to64(p):
    out = {k: (v.astype(np.float64) if isinstance(v, np.ndarray) else v) for k, v in p.items()}
    out["layers"] = [{k: v.astype(np.float64) for k, v in L.items()} for L in p["layers"]]
    return out


@pytest.mark.parametrize("seed", [80, 81])
def test_encoder_against_float64(seed):
    p = make(ENC, seed)
    mel = synth.activations(seed, 2 * ENC["positions"], ENC["mels"])
    got = oracle_encoder(ENC, p).encode(mel)
    p64 = to64(p)
    err = rel(got, W.encode(ENC, p64, mel.astype(np.float64)))
    print(f"encoder: {err:.3g}")
    assert err < TOL
    for mistake in MISTAKES:
        bad = rel(got, W.encode(ENC, p64, mel.astype(np.float64), mistake))
        print(f"  planted {mistake}: {bad:.3g}")
        assert bad > MISTAKE_TOL, mistake
