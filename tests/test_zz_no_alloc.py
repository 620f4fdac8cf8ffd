"""trit_hip_layer_forward_device_noalloc against trit_hip_layer_forward_device:
the same layers and device inputs through both, bit for bit, on two calls in a
row (the second with fewer rows, so the array keeps the first call's larger
contents), for the matrix-core product (many rows), the small-batch image of
2..8 rows (32- and 128-groups) and one row; and a product too large for the
array fails with an error naming the bytes it needs."""

import numpy as np
import pytest

from tests.device_memory import Device
from trit_amd import hip, synth

pytestmark = pytest.mark.gpu


def both(D, layer, x_dev, m, relu=0):
    """The product through the allocating entry point and the no-allocation one."""
    lib = hip.lib()
    y_ref = D.empty(m * layer.n * 4)
    y_new = D.empty(m * layer.n * 4)
    hip.check(lib.trit_hip_layer_forward_device(layer.h, x_dev, m, relu, y_ref, None))
    hip.check(lib.trit_hip_layer_forward_device_noalloc(layer.h, x_dev, m, relu, y_new, None))
    return D.download(y_ref, (m, layer.n)), D.download(y_new, (m, layer.n))


def same_bits(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_matches_the_allocating_forward(gpu):
    D = Device()
    try:
        n = k = 2048
        codes, sbits = synth.q8_0_matrix(synth.seed_for(9, 1), n, k)
        q8 = hip.Dense.q8_0(n, k, synth.q8_0_blocks(codes, sbits))
        x = D.upload(synth.activations(synth.seed_for(9, 2), 1564, k))
        # 1564 rows: the matrix-core product (its quantized rows take 3.6 MB
        # of the array), then 5 rows: the small-batch image over the stale
        # rest, then one row.
        for m in (1564, 5, 1):
            ref, got = both(D, q8, x, m)
            assert same_bits(ref, got), f"Q8_0 {m} rows"
            print(f"Q8_0 {n}x{k}, {m} rows: bit-exact")
        # 128-groups: ternary at 8 rows, then 3.
        tcodes, tscales = synth.ternary_matrix(synth.seed_for(9, 3), 1024, 4096)
        tern = hip.Dense.ternary(tcodes, tscales)
        xt = D.upload(synth.activations(synth.seed_for(9, 4), 8, 4096))
        for m in (8, 3):
            ref, got = both(D, tern, xt, m)
            assert same_bits(ref, got), f"ternary {m} rows"
            print(f"ternary 1024x4096, {m} rows: bit-exact")
        # A product whose quantized rows exceed the array is refused before any launch.
        lib = hip.lib()
        big = hip.Dense.q8_0(128, 8192, synth.q8_0_blocks(*synth.q8_0_matrix(synth.seed_for(9, 5), 128, 8192)))
        xb = D.empty(600 * 8192 * 4)
        yb = D.empty(600 * 128 * 4)
        assert lib.trit_hip_layer_forward_device_noalloc(big.h, xb, 600, 0, yb, None) == -1
        msg = lib.trit_hip_last_error().decode()
        assert "bytes of scratch" in msg and "4194304" in msg, msg
        for layer in (q8, tern, big):
            layer.free()
    finally:
        D.free()
