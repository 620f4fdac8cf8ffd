"""The oracle's Qwen3-ASR audio encoder (AudioEncoder::encode and ::chunk,
src/models/families/qwen3_asr.rs:321-405) pinned: the sinusoid table
against its closed form and known values, the 2-D im2col against direct
indexing, and the composition (chunks, padding, convolutions, the
channel-major columns, positions, windowed attention, projections) against
a float64 encoder written from the model definition, with planted mistakes
that the check catches."""

import math

import numpy as np
import pytest

from oracle import oracle as O
from tests import qwen3_asr_float64 as A
from trit_amd import synth

# 108 frames: chunks of 32, 32, 32 and 12 frames (4, 4, 4 and 2 rows),
# windows of 8 rows.
ASR = dict(d=64, layers=2, heads=4, ffn=128, mels=16, channels=8, chunk=32, window_chunks=2, out=48,
           max_positions=40)
FRAMES = 108
TOL = 2e-5  # of the largest output: f32 against float64
MISTAKE_TOL = 10 * TOL
MISTAKES = ["taps_transposed", "bin_major", "global_attention", "positions_offset", "pad_own_length"]


def test_sinusoids_known_values():
    d = 64
    t = O.sinusoids(50, d)
    assert np.array_equal(t[0, :32], np.zeros(32, np.float32))
    assert np.array_equal(t[0, 32:], np.ones(32, np.float32))
    for p in (1, 7, 49):
        assert t[p, 0] == np.float32(math.sin(p)) and t[p, 32] == np.float32(math.cos(p))
        # The last frequency is 1/10000: the exponent's denominator is d/2 - 1.
        assert abs(t[p, 31] - math.sin(p / 10000.0)) < 1e-7
    want = A.sinusoids(50, d)
    assert np.max(np.abs(t - want)) < 1e-6


def test_conv2d_columns_direct():
    bins, times, ch = 7, 6, 3
    m = synth.activations(320, bins * times, ch)
    got = O.conv2d_columns(m, bins, times, ch)
    ob, ot = 4, 3
    assert got.shape == (ob * ot, ch * 9)
    for y in range(ob):
        for x in range(ot):
            for dy in range(3):
                for dx in range(3):
                    sy, sx = 2 * y + dy - 1, 2 * x + dx - 1
                    want = m[sy * times + sx] if 0 <= sy < bins and 0 <= sx < times else np.zeros(ch, np.float32)
                    assert np.array_equal(got[y * ot + x, 3 * dy + dx::9], want)


def make(cfg, seed):
    """Random f32 weights for both sides."""
    d, ffn, ch, out = cfg["d"], cfg["ffn"], cfg["channels"], cfg["out"]
    bins = cfg["mels"]
    for _ in range(3):
        bins = (bins + 1) // 2
    t = [0]

    def mat(*shape):
        t[0] += 1
        fan = int(np.prod(shape[1:]))
        return (synth.normal(synth.seed_for(seed, t[0]), shape) / np.sqrt(fan)).astype(np.float32)

    def vec(n, base=0.0, spread=0.2):
        t[0] += 1
        return (base + spread * (2 * synth.uniform(synth.seed_for(seed, t[0]), n) - 1)).astype(np.float32)

    p = dict(convs=[(mat(ch, 1, 3, 3), vec(ch)), (mat(ch, ch, 3, 3), vec(ch)), (mat(ch, ch, 3, 3), vec(ch))],
             conv_out=(mat(d, ch * bins), vec(d)), post_w=vec(d, 1.0), post_b=vec(d),
             proj1=(mat(d, d), vec(d)), proj2=(mat(out, d), vec(out)), layers=[])
    for _ in range(cfg["layers"]):
        p["layers"].append(dict(q=mat(d, d), k=mat(d, d), v=mat(d, d), o=mat(d, d), fc1=mat(ffn, d),
                                fc2=mat(d, ffn), bq=vec(d), bk=vec(d), bv=vec(d), bo=vec(d), b1=vec(ffn),
                                b2=vec(d), attn_w=vec(d, 1.0), attn_b=vec(d), ffn_w=vec(d, 1.0), ffn_b=vec(d)))
    return p


def oracle_encoder(cfg, p):
    """O.AsrEncoder with f32 products; conv weights as [out][in * 9]."""

    def f32(w, b):
        w = np.ascontiguousarray(w.reshape(w.shape[0], -1), np.float32)
        return lambda x: (O.matmul_f32(np.ascontiguousarray(x, np.float32), w) + b).astype(np.float32)

    products = [f32(w, b) for w, b in p["convs"]] + [f32(*p["conv_out"])]
    norms = []
    for L in p["layers"]:
        qkv = np.concatenate([L["q"], L["k"], L["v"]])
        bqkv = np.concatenate([L["bq"], L["bk"], L["bv"]])
        products += [f32(qkv, bqkv), f32(L["o"], L["bo"]), f32(L["fc1"], L["b1"]), f32(L["fc2"], L["b2"])]
        norms += [L["attn_w"], L["attn_b"], L["ffn_w"], L["ffn_b"]]
    products += [f32(*p["proj1"]), f32(*p["proj2"])]
    norms += [p["post_w"], p["post_b"]]
    return O.AsrEncoder(cfg, products, norms)


def to64(p):
    pair = lambda wb: (wb[0].astype(np.float64), wb[1].astype(np.float64))
    return dict(convs=[pair(c) for c in p["convs"]], conv_out=pair(p["conv_out"]), proj1=pair(p["proj1"]),
                proj2=pair(p["proj2"]), post_w=p["post_w"].astype(np.float64), post_b=p["post_b"].astype(np.float64),
                layers=[{k: v.astype(np.float64) for k, v in L.items()} for L in p["layers"]])


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def test_rows():
    enc = O.AsrEncoder(ASR, [], [])
    assert enc.rows(FRAMES) == 14
    assert enc.rows(32) == 4 and enc.rows(1) == 1 and enc.rows(33) == 5


@pytest.mark.parametrize("seed", [90, 91])
def test_asr_encoder_against_float64(seed):
    p = make(ASR, seed)
    mel = synth.activations(seed, FRAMES, ASR["mels"])
    got = oracle_encoder(ASR, p).encode(mel, FRAMES)
    assert got.shape == (14, ASR["out"])
    p64 = to64(p)
    err = rel(got, A.encode(ASR, p64, mel.astype(np.float64), FRAMES))
    print(f"asr encoder: {err:.3g}")
    assert err < TOL
    for mistake in MISTAKES:
        bad = rel(got, A.encode(ASR, p64, mel.astype(np.float64), FRAMES, mistake))
        print(f"  planted {mistake}: {bad:.3g}")
        assert bad > MISTAKE_TOL, mistake
