"""GPU products against the oracle, bit for bit (integer dots and f32 outputs).

Each case prints its name before it runs, so a failing GPU step names itself.
"""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import synth

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def q8_layer(seed, n, k, scale="uniform"):
    codes, sbits = synth.q8_0_matrix(seed, n, k, scale=scale)
    return codes, sbits, synth.q8_0_blocks(codes, sbits)


@pytest.mark.parametrize("n,k,m", [(2048, 2048, 1), (4096, 1024, 1), (1024, 2048, 1), (6144, 1024, 1),
                                   (1024, 3072, 1), (2048, 2048, 8), (4096, 1024, 3), (32, 32, 1),
                                   (96, 160, 5), (1024, 8192, 2)])
def test_q8_0(gpu, n, k, m):
    print(f"case q8_0 n={n} k={k} m={m}", flush=True)
    codes, sbits, blocks = q8_layer(synth.seed_for(1, n + k), n, k)
    x = synth.activations(synth.seed_for(1, 7 + m), m, k)
    ref = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x)
    layer = gpu.Dense.q8_0(n, k, blocks)
    got = layer.forward(x)
    assert bits_equal(got, ref), np.max(np.abs(got - ref))


# Products of a few tens of MB and 2..8 rows run on the streaming kernel
# (persistent waves, segments of 1024 inputs); same bits.
@pytest.mark.parametrize("n,k,m", [(16384, 3072, 1), (3072, 8192, 1), (4096, 3072, 4), (4096, 4096, 7),
                                   (8192, 2048, 8), (12288, 1024, 3)])
def test_q8_0_stream(gpu, n, k, m):
    print(f"case q8_0 stream n={n} k={k} m={m}", flush=True)
    codes, sbits, blocks = q8_layer(synth.seed_for(3, n + k), n, k)
    x = synth.activations(synth.seed_for(3, 7 + m), m, k)
    ref = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x)
    got = gpu.Dense.q8_0(n, k, blocks).forward(x)
    assert bits_equal(got, ref), np.max(np.abs(got - ref))


def test_q8_0_stream_bias_relu(gpu):
    n, k = 2048, 4096
    codes, sbits, blocks = q8_layer(14, n, k)
    bias = synth.activations(15, 1, n)[0]
    for m in (1, 3):
        print(f"case q8_0 stream bias relu m={m}", flush=True)
        x = synth.activations(16 + m, m, k)
        ref = np.maximum(O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x) + bias, 0)
        got = gpu.Dense.q8_0(n, k, blocks, bias).forward(x, relu=True)
        assert bits_equal(got, ref)


def test_q8_0_bias_relu(gpu):
    n, k = 256, 512
    codes, sbits, blocks = q8_layer(11, n, k)
    bias = synth.activations(12, 1, n)[0]
    x = synth.activations(13, 2, k)
    ref = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x) + bias
    ref = np.maximum(ref, 0)
    got = gpu.Dense.q8_0(n, k, blocks, bias).forward(x, relu=True)
    assert bits_equal(got, ref)


# More than 8 rows: the matrix-core product (int8 MFMA), same bits.
@pytest.mark.parametrize("n,k,m", [(256, 512, 9), (384, 1024, 64), (128, 256, 100), (2048, 2048, 257),
                                   (1024, 3072, 40), (128, 384, 70), (256, 4320, 33), (128, 32, 12),
                                   (384, 1248, 129), (480, 4320, 70), (32, 256, 40), (224, 512, 65), (96, 96, 17)])
def test_q8_0_many_rows(gpu, n, k, m):
    print(f"case q8_0 matrix cores n={n} k={k} m={m}", flush=True)
    codes, sbits, blocks = q8_layer(synth.seed_for(2, n + k), n, k)
    x = synth.activations(synth.seed_for(2, 7 + m), m, k)
    ref = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x)
    got = gpu.Dense.q8_0(n, k, blocks).forward(x)
    assert bits_equal(got, ref), np.max(np.abs(got - ref))


@pytest.mark.parametrize("n", [256, 224])
def test_q8_0_many_rows_bias_relu(gpu, n):
    print(f"case q8_0 matrix cores bias relu n={n}", flush=True)
    k, m = 512, 33
    codes, sbits, blocks = q8_layer(14, n, k)
    bias = synth.activations(15, 1, n)[0]
    x = synth.activations(16, m, k)
    ref = np.maximum(O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x) + bias, 0)
    got = gpu.Dense.q8_0(n, k, blocks, bias).forward(x, relu=True)
    assert bits_equal(got, ref)


@pytest.mark.parametrize("n", [2048, 6144])
def test_prefill_gemm_1564_rows(gpu, n):
    """The audio-LLM prefill contraction: 1500 encoder + 64 text rows, K 2048.
    The oracle checks a sample of rows (each output row depends on its own
    input row only), the edges of the 64-row tiles included."""
    print(f"case q8_0 prefill 1564x2048 n={n}", flush=True)
    m, k = 1564, 2048
    codes, sbits, blocks = q8_layer(synth.seed_for(5, n), n, k)
    x = synth.activations(synth.seed_for(5, 1564), m, k)
    got = gpu.Dense.q8_0(n, k, blocks).forward(x)
    rows = sorted(set([0, 1, 31, 32, 63, 64, 127, 1499, 1500, 1535, 1536, 1562, 1563]
                      + synth.ints(55, (19,), 0, m - 1).tolist()))
    ref = O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True)(x[rows])
    assert bits_equal(got[rows], ref), np.max(np.abs(got[rows] - ref))
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("n,k,m", [(512, 1024, 1), (384, 2048, 4), (256, 512, 33), (512, 1024, 70), (256, 384, 40),
                                   (128, 128, 20), (480, 384, 30)])
def test_int8(gpu, n, k, m):
    print(f"case int8 n={n} k={k} m={m}", flush=True)
    codes = synth.ints(21, (n, k), -127, 127).astype(np.int8)
    scales = (0.001 + 0.01 * synth.uniform(22, (n, k // 128))).astype(np.float32)
    x = synth.activations(23, m, k)
    ref = O.Int8(codes, scales, 128, False)(x)
    got = gpu.Dense.int8(codes, scales).forward(x)
    assert bits_equal(got, ref)


def ternary_inputs(n, k):
    u = synth.uniform(31, (n, k))
    codes = np.where(u < 0.25, 0, np.where(u < 0.75, 1, 2)).astype(np.uint8)
    row_scale = (0.01 + 0.04 * synth.uniform(32, (n, 1))).astype(np.float32)
    scales = np.repeat(row_scale, k // 128, axis=1)
    return codes, scales


@pytest.mark.parametrize("m", [1, 8, 12])
def test_ternary_4096(gpu, m):
    print(f"case ternary 4096x4096 m={m}", flush=True)
    n = k = 4096
    codes, scales = ternary_inputs(n, k)
    x = synth.activations(33 + m, m, k)
    ref = O.Ternary(codes, scales)(x)
    got = gpu.Dense.ternary(codes, scales).forward(x)
    assert bits_equal(got, ref)


# The streaming kernel's ternary form (k a multiple of 2048), 1..8 rows.
# (2048, 2048, 8): 8 rows of 2048 inputs quantize inside each block.
@pytest.mark.parametrize("n,k,m", [(2048, 2048, 1), (8192, 4096, 3), (1024, 6144, 8), (4096, 2048, 2),
                                   (2048, 2048, 8), (4096, 2048, 5)])
def test_ternary_stream(gpu, n, k, m):
    print(f"case ternary stream n={n} k={k} m={m}", flush=True)
    codes, scales = ternary_inputs(n, k)
    # A scale per (row, 128-group), so that a wrong group index shows.
    scales = (scales * (0.5 + synth.uniform(37, scales.shape))).astype(np.float32)
    x = synth.activations(36 + m, m, k)
    ref = O.Ternary(codes, scales)(x)
    got = gpu.Dense.ternary(codes, scales).forward(x)
    assert bits_equal(got, ref)


@pytest.mark.parametrize("n,k,m", [(1024, 4096, 6), (2048, 4096, 8), (4096, 2048, 8)])
def test_stream_after_quantization_pass(gpu, monkeypatch, n, k, m):
    """TRIT_HIP_GEMV_STREAM=1: 5..8 rows too many to quantize in the block
    run on the streaming kernel from the quantization pass's image (below
    the size where it is chosen by itself), ternary and Q8_0."""
    print(f"case stream after the quantization pass n={n} k={k} m={m}", flush=True)
    monkeypatch.setenv("TRIT_HIP_GEMV_STREAM", "1")
    codes, scales = ternary_inputs(n, k)
    x = synth.activations(38 + m, m, k)
    assert bits_equal(gpu.Dense.ternary(codes, scales).forward(x), O.Ternary(codes, scales, O.isa_best())(x))
    qc, sbits, blocks = q8_layer(synth.seed_for(6, n + k), n, k)
    ref = O.Int8(qc, sbits.view(np.float16).astype(np.float32), 32, True, O.isa_best())(x)
    assert bits_equal(gpu.Dense.q8_0(n, k, blocks).forward(x), ref)


def test_ternary_base3(gpu):
    n, k = 64, 640
    codes, scales = ternary_inputs(n, k)
    row_bytes = (k + 4) // 5
    packed = np.zeros((n, row_bytes), np.uint8)
    for d in range(5):
        idx = np.arange(row_bytes) * 5 + d
        valid = idx < k
        packed[:, valid] += (codes[:, idx[valid]] * 3 ** d).astype(np.uint8)
    x = synth.activations(35, 2, k)
    ref = O.Ternary(codes, scales)(x)
    got = gpu.Dense.ternary_base3(n, k, packed, scales).forward(x)
    assert bits_equal(got, ref)


# The 3B layer set of the Q4_K configuration (Wqkv 3072 -> 4096, Wo 3072 ->
# 3072, gate/up 3072 -> 16384, down 8192 -> 3072) at 1 to 4 rows, and small
# shapes through the tiled and matrix-core kernels. Each layer is made with
# TRIT_HIP_Q4K=1 (it keeps its super-blocks); each case runs the native
# product (1..4 rows) and, with TRIT_HIP_Q4K=0 at the call, the products on
# Trit's requantized Q8_0 codes.
@pytest.mark.parametrize("n,k,m", [(4096, 3072, 1), (4096, 3072, 4), (3072, 3072, 1), (3072, 3072, 4),
                                   (16384, 3072, 1), (16384, 3072, 4), (3072, 8192, 1), (3072, 8192, 4),
                                   (3072, 8192, 2), (4096, 3072, 3), (512, 256, 1), (768, 1024, 2),
                                   (256, 512, 3), (256, 512, 20)])
def test_q4_k(gpu, n, k, m, monkeypatch):
    blocks = synth.q4_k_blocks(41 + n, n, k)
    vals = O.q4_k_expand(blocks)
    codes, scales = O.q8_0_quantize(vals)
    x = synth.activations(42 + m, m, k)
    ref = O.Int8(codes.reshape(n, k), scales.reshape(n, k // 32), 32, True, O.isa_best())(x)
    monkeypatch.setenv("TRIT_HIP_Q4K", "1")
    layer = gpu.Dense.q4_k(n, k, blocks)
    assert layer.info()["bytes"] == n * k + n * k // 32 * 2 + n * k // 256 * 144
    for mode in ("1", "0"):
        print(f"case q4_k n={n} k={k} m={m} native={mode}", flush=True)
        monkeypatch.setenv("TRIT_HIP_Q4K", mode)
        got = layer.forward(x)
        assert bits_equal(got, ref), mode


def same_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


def test_q4_k_non_finite_blocks(gpu, monkeypatch):
    """Super-blocks whose d or dmin is infinite or NaN: their codes follow
    Trit's expression (Rust's `as i8`: NaN codes 0), on the native product
    and on the requantized codes alike; the rows they reach are NaN or
    infinite in both (NaN payloads aside)."""
    n, k = 512, 1024
    blocks = synth.q4_k_blocks(44, n, k).reshape(n, k // 256, 144).copy()
    half = lambda v: np.array([v], np.float16).view(np.uint8)
    blocks[3, 1, 0:2] = half(np.inf)          # d infinite
    blocks[70, 2, 2:4] = half(np.nan)         # dmin NaN
    blocks[100, 0, 0:2] = half(-np.inf)       # d -inf
    blocks[101, 3, 0:4] = np.concatenate([half(np.inf), half(np.inf)])  # both infinite
    blocks[200, 1, 0:2] = half(0.0)           # d 0: codes from the mins alone
    blocks = blocks.reshape(-1)
    vals = O.q4_k_expand(blocks)
    codes, scales = O.q8_0_quantize(vals)
    monkeypatch.setenv("TRIT_HIP_Q4K", "1")
    layer = gpu.Dense.q4_k(n, k, blocks)
    for m in (1, 3):
        x = synth.activations(45 + m, m, k)
        ref = O.Int8(codes.reshape(n, k), scales.reshape(n, k // 32), 32, True, O.isa_best())(x)
        for mode in ("1", "0"):
            print(f"case q4_k non-finite m={m} native={mode}", flush=True)
            monkeypatch.setenv("TRIT_HIP_Q4K", mode)
            got = layer.forward(x)
            assert same_or_both_nan(got, ref), mode


@pytest.mark.parametrize("n,k,m", [(4096, 1024, 1), (1000, 1024, 3), (300, 2048, 2), (77, 160, 5), (300, 384, 8),
                                   (65, 3072, 6), (100, 8192, 3), (480, 9, 8), (33, 71, 4), (480, 9, 130), (40, 64, 70)])
def test_f16(gpu, n, k, m):
    print(f"case f16 n={n} k={k} m={m}", flush=True)
    w = synth.f16_bits(synth.activations(51 + n, n, k) * 0.02).reshape(n, k)
    x = synth.activations(52 + m, m, k)
    ref = O.matmul_f16(x, w)
    layer = gpu.Dense.f16(w)
    got = layer.forward(x)
    assert bits_equal(got, ref)
    row = layer.row(n // 2)
    assert np.array_equal(row, w[n // 2].view(np.float16).astype(np.float32))


def widened_q8(codes, scales):
    """widen_q8 (src/cpu/gemm.rs:171-179): f32(code) * its 32-group's scale,
    one f32 rounding."""
    return codes.astype(np.float32) * np.repeat(np.asarray(scales, np.float32), 32, axis=1)


@pytest.mark.parametrize("n,k,m", [(300, 1024, 1), (77, 160, 5), (1280, 1280, 5), (100, 4096, 8), (4096, 2048, 2),
                                   (33, 48, 3), (480, 9, 8), (70, 1, 3), (50, 37, 5), (100, 300, 2), (480, 9, 300),
                                   (70, 100, 65), (300, 128, 9), (33, 17, 12)])
def test_f32(gpu, n, k, m):
    print(f"case f32 n={n} k={k} m={m}", flush=True)
    w = synth.activations(61 + n, n, k) * np.float32(0.05)
    bias = synth.activations(62 + n, 1, n)[0]
    x = synth.activations(63 + m, m, k)
    layer = gpu.Dense.f32(w, bias)
    assert bits_equal(layer.forward(x), O.matmul_f32(x, w) + bias)
    assert np.array_equal(layer.row(n - 1), w[n - 1])


@pytest.mark.parametrize("n,k,m", [(300, 1024, 1), (77, 160, 5), (1280, 1280, 5), (96, 4096, 8), (5000, 1024, 1),
                                   (40, 96, 2), (40, 96, 20)])
def test_q8_table(gpu, n, k, m):
    """Weights::Q8 (int8 storage, f32 scale per 32, f32 math)."""
    print(f"case q8 n={n} k={k} m={m}", flush=True)
    codes = synth.ints(71 + n, (n, k), -127, 127).astype(np.int8)
    scales = (np.abs(synth.activations(72 + n, n, k // 32)) * np.float32(0.01)).astype(np.float32)
    x = synth.activations(73 + m, m, k)
    layer = gpu.Dense.q8(codes, scales)
    w = widened_q8(codes, scales)
    assert bits_equal(layer.forward(x), O.matmul_f32(x, w))
    assert bits_equal(layer.row(n // 3), w[n // 3])


@pytest.mark.parametrize("n,k,m,table", [(100, 256, 3, False), (1000, 1024, 1, True), (64, 512, 4, True)])
def test_q8_0_f32_math(gpu, n, k, m, table):
    """Q8_0 blocks with f32 math: a layer whose n is no multiple of 32
    (Dense::q8_0 outside Int8::fits_group) and a token table (Dense::table
    under Q8_0): the codes times the widened f16 block scales."""
    print(f"case q8_0 f32 math n={n} k={k} m={m} table={table}", flush=True)
    codes, sbits, blocks = q8_layer(synth.seed_for(2, n + k), n, k)
    x = synth.activations(74 + m, m, k)
    layer = gpu.Dense.q8_0_f32(n, k, blocks) if table else gpu.Dense.q8_0(n, k, blocks)
    assert layer.info()["kind"] == gpu.Q8
    w = widened_q8(codes, sbits.view(np.float16).astype(np.float32).reshape(n, k // 32))
    assert bits_equal(layer.forward(x), O.matmul_f32(x, w))


@pytest.mark.parametrize("ggml_type", [2, 3, 6, 7, 12, 13, 14])
@pytest.mark.parametrize("n,k,m,f32_math", [(512, 512, 1, False), (256, 1024, 5, False), (96, 256, 3, True),
                                            (100, 512, 2, False)])
def test_ggml_types(gpu, ggml_type, n, k, m, f32_math):
    """ggml's other block types as Trit loads them: expanded as ggml does and
    requantized to Q8_0 (the oracle's expansion, then Blocks::quantize),
    then int8 activations, or f32 math for a table or an n that is no
    multiple of 32."""
    print(f"case ggml type {ggml_type} n={n} k={k} m={m} f32_math={f32_math}", flush=True)
    blocks = synth.ggml_blocks(synth.seed_for(3, ggml_type * 7 + n), ggml_type, n, k)
    codes, scales = O.q8_0_quantize(O.ggml_expand(ggml_type, blocks))
    codes = codes.reshape(n, k)
    scales = scales.reshape(n, k // 32)
    x = synth.activations(81 + m, m, k)
    layer = gpu.Dense.ggml(n, k, ggml_type, blocks, f32_math=f32_math)
    if f32_math or n % 32:
        assert layer.info()["kind"] == gpu.Q8
        want = O.matmul_f32(x, widened_q8(codes, scales))
    else:
        want = O.Int8(codes, scales, 32, True)(x)
    assert bits_equal(layer.forward(x), want)


def test_f16_conversions(gpu):
    """The device's f16 conversions against the oracle's (Trit's f32_to_f16 /
    f16_to_f32): all 65536 f16 patterns; every f32 value where rounding to
    f16 can turn (each f16 value, each midpoint and its neighbours, both
    signs, the subnormal steps and the overflow edge); and every 4093rd of
    the 2^32 f32 patterns. Bit for bit but NaN, which stays NaN."""
    print("case f16 conversions", flush=True)
    h = np.arange(65536, dtype=np.uint16)
    got, want = gpu.f16_to_f32(h), O.f16_to_f32(h)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.all(np.isnan(got[nan]))
    sweep = (np.arange(0, 1 << 32, 4093, dtype=np.uint64)).astype(np.uint32).view(np.float32)
    for v in (O.f16_boundaries(), sweep):
        got, want = gpu.f32_to_f16(v), O.f32_to_f16(v)
        nan = np.isnan(v)
        assert np.array_equal(got[~nan], want[~nan])
        assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x03FF) != 0)


def test_errors(gpu):
    from trit_amd.hip import TritError

    with pytest.raises(TritError, match="multiple of 32"):
        gpu.Dense.q8_0(32, 48, np.zeros(32 * 48 // 32 * 34 + 34, np.uint8)[: 32 * 48 // 32 * 34])
    with pytest.raises(TritError, match="does not exist"):
        gpu.init(99)
