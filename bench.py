"""Decode throughput of Trit's token loop on one MI355X.

Workload (the reference's full-loop configuration): a Qwen3-0.6B-shape
decoder (28 layers, d 1024, 16/8 heads x 128, SwiGLU 3072, vocab 151936,
tied f16 head) with random Q8_0 weights (codes uniform in [-127, 127],
block scales N(0, 0.02)/127) and f16 embeddings N(0, 0.02); a 256-token
random prompt is prefilled, then 128 greedy steps run. A "step" is one
greedy decode token. `value` is decode tokens/s with every weight resident
in HBM before the timed region.

The JSON line also carries
- roofline: the dominant decode product (the Q8_0 gate_up weights, 6144 x
  1024, one row) timed with HIP events stamped at the kernel's start and
  end, launch by launch, inside sweeps over all 112 Q8_0 products of a step
  in decode order (so its weights come from HBM, not the 256 MB Infinity
  Cache);
- cpu_baseline: the oracle (a C++ restatement of Trit's AVX-512 VNNI path,
  one pinned thread per core of the largest L3 domain) on the same weights
  and prompt, with the greedy tokens of both compared.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from trit_amd import hip, model, synth  # noqa: E402

METRIC = "decode tokens/sec + GEMV HBM GB/s (% of peak), Qwen3-0.6B-shape Q8_0, 1 GPU"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
# Vector ALU lane operations per second: MI355X's published FP32 vector rate,
# 157.3 TFLOP/s, is 78.6 T lane FMAs/s (256 CUs x 128 lanes a cycle x 2.4 GHz;
# a wave64 f32 instruction issues every 2 cycles a SIMD). A loop of the exact
# chain's operations (convert, multiply, FMA, and an integer add, over 32
# independent values a lane, no memory) ran at 63.7 T/s with the clock at
# 2.27 GHz.
VALU_PEAK_TOPS = 78.64
# HBM bytes per launch of the roofline kernel, from rocprofv3 --pmc runs of
# `bench.py --profile-pass` (profiles/gemv_stream_q8_0_6144x1024_hbm_traffic.md):
# FETCH_SIZE 3353.1 KiB x 2.0 (the scale a 256 MiB device copy gives) plus
# WRITE_SIZE 24.0 KiB x 1.0.
GATE_UP_TRAFFIC_BYTES = round((3353.1 * 2.0 + 24.0) * 1024)
# HBM bytes per forward of the persistent decode step, from the same kind of
# runs (profiles/decode_step_qwen3_0.6b_hbm_traffic.md): FETCH_SIZE and
# WRITE_SIZE of one launch of 128 steps (127 forwards, positions 256..382)
# over the forwards, FETCH_SIZE x 2.0 plus WRITE_SIZE x 1.0; the default
# mode (f16 caches) and the exact mode (f32 caches).
STEP_FETCH_KIB, STEP_WRITE_KIB = 51636554.562500 / 127, 222703.812500 / 127
STEP_TRAFFIC_BYTES = round((STEP_FETCH_KIB * 2.0 + STEP_WRITE_KIB) * 1024)
EXACT_FETCH_KIB, EXACT_WRITE_KIB = 54617490.937500 / 127, 1644912.000000 / 127
EXACT_TRAFFIC_BYTES = round((EXACT_FETCH_KIB * 2.0 + EXACT_WRITE_KIB) * 1024)


class Hip:
    """The few HIP runtime calls the timing needs."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        for name in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                     "hipMalloc", "hipFree", "hipStreamCreate", "hipStreamSynchronize", "hipMemcpy"):
            getattr(self.L, name).restype = C.c_int

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def stream(self):
        s = C.c_void_p()
        self.ok(self.L.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s

    def event(self):
        e = C.c_void_p()
        self.ok(self.L.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e

    def record(self, e, s):
        self.ok(self.L.hipEventRecord(e, s), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ok(self.L.hipEventSynchronize(b), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.L.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def malloc(self, nbytes):
        p = C.c_void_p()
        self.ok(self.L.hipMalloc(C.byref(p), C.c_size_t(nbytes)), "hipMalloc")
        return p

    def upload(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self.ok(self.L.hipMemcpy(dst, arr.ctypes.data_as(C.c_void_p), C.c_size_t(arr.nbytes), 1), "hipMemcpy")

    def sync(self, s):
        self.ok(self.L.hipStreamSynchronize(s), "hipStreamSynchronize")


def build_layers(w):
    cfg = w.cfg
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    qkv_rows = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    linears = []
    for L in w.layers:
        linears += [hip.Dense.q8_0(qkv_rows, d, L.qkv), hip.Dense.q8_0(d, cfg["heads"] * hd, L.o),
                    hip.Dense.q8_0(2 * ffn, d, L.gate_up), hip.Dense.q8_0(d, ffn, L.down)]
    embed = hip.Dense.f16(w.embed)
    lm = hip.CausalLm(cfg, linears, w.norms_packed(), embed)
    return lm, linears, embed


def gemv_roofline(H, linears, cfg, sweeps):
    """HIP-event duration of each gate_up product inside decode-order sweeps."""
    stream = H.stream()
    d, ffn = cfg["d"], cfg["ffn"]
    width = max(d, ffn, cfg["heads"] * cfg["head_dim"], 2 * ffn + 64)
    x = H.malloc(width * 4)
    y = H.malloc(width * 4 * 2)
    H.upload(x, synth.activations(synth.seed_for(1, 999), 1, width)[0])
    fwd = hip.lib().trit_hip_layer_forward_device
    timed = hip.lib().trit_hip_layer_forward_timed
    durations = []
    events = [(H.event(), H.event()) for _ in range(len(linears) // 4)]
    for sweep in range(sweeps + 1):
        for i, layer in enumerate(linears):
            if i % 4 == 2:
                # The gate_up weights as a plain layer product (one kernel launch).
                a, b = events[i // 4]
                hip.check(timed(layer.h, x, 1, 0, y, stream, a, b))
            else:
                hip.check(fwd(layer.h, x, 1, 0, y, stream))
        H.sync(stream)
        if sweep > 0:  # the first sweep warms up
            durations += [H.elapsed_ms(a, b) for a, b in events]
    avg_ms = float(np.mean(durations))
    # Algorithmic bytes of one launch: the Q8_0 blocks (34 bytes per 32
    # weights), the f32 input row and the f32 output row.
    weight = 2 * ffn * d * 34 // 32
    algo = weight + d * 4 + 2 * ffn * 4
    achieved = algo / (avg_ms * 1e-3) / 1e9
    return dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBS, 4), traffic=GATE_UP_TRAFFIC_BYTES,
                kernel="gemv_stream_kernel<Q8S,1,1,4>: Q8_0 one-row product, the 6144x1024 gate_up weights",
                bytes_per_launch=algo, avg_us=round(avg_ms * 1e3, 3), launches=len(durations),
                timing="hipExtLaunchKernel start/stop events per launch, inside decode-order sweeps of "
                       "all 112 Q8_0 products (468 MB per sweep, past the 256 MB Infinity Cache)")


def timed_sweeps(H, stream, layers, x, y, m, sweeps):
    """Average kernel time (ms) of each product launch, stamped by HIP events
    at the kernel's start and end, over `sweeps` passes through `layers`
    (copies of the weights whose total exceeds the Infinity Cache)."""
    timed = hip.lib().trit_hip_layer_forward_timed
    events = [(H.event(), H.event()) for _ in layers]
    durations = []
    for sweep in range(sweeps + 1):
        for (a, b), layer in zip(events, layers):
            hip.check(timed(layer.h, x, m, 0, y, stream, a, b))
        H.sync(stream)
        if sweep > 0:
            durations += [H.elapsed_ms(a, b) for a, b in events]
    return float(np.mean(durations))


def back_to_back(H, stream, layers, x, y, m, sweeps):
    """Average time (ms) per product when `layers` run back to back on one
    stream with no per-launch events: one event pair around `sweeps` passes
    (the rate of a sequence of products, launch overheads overlapped)."""
    fwd = hip.lib().trit_hip_layer_forward_device
    for layer in layers:
        hip.check(fwd(layer.h, x, m, 0, y, stream))
    a, b = H.event(), H.event()
    H.record(a, stream)
    for _ in range(sweeps):
        for layer in layers:
            hip.check(fwd(layer.h, x, m, 0, y, stream))
    H.record(b, stream)
    H.sync(stream)
    return H.elapsed_ms(a, b) / (sweeps * len(layers))


def config_lines(H, sweeps=10, decode=True):
    """The per-product configurations: C1 Q8_0 GEMV, C3 ternary GEMV, C4
    Q4_K set, C5 prefill GEMM on the matrix cores; then (decode) the decode
    loops of the other workloads."""
    stream = H.stream()
    out = {}
    xbuf = H.malloc(1564 * 8192 * 4)
    ybuf = H.malloc(1564 * 16384 * 4)
    H.upload(xbuf, synth.activations(synth.seed_for(0, 77), 64, 8192))

    def gbs(nbytes, ms):
        return round(nbytes / (ms * 1e-3) / 1e9, 1)

    # The floor of one timed product: a 64 x 1024 Q8_0 product (68 KB of
    # weights), 64 copies, by the same per-launch events -- launch, the
    # activation and weight latencies and the store, next to no streaming.
    codes, sbits = synth.q8_0_matrix(synth.seed_for(0, 2), 64, 1024)
    tiny = [hip.Dense.q8_0(64, 1024, synth.q8_0_blocks(codes, sbits)) for _ in range(64)]
    floor_ms = timed_sweeps(H, stream, tiny, xbuf, ybuf, 1, sweeps)
    out["product_floor_q8_0_64x1024_b1"] = dict(
        avg_us=round(floor_ms * 1e3, 3), back_to_back_us=round(back_to_back(H, stream, tiny, xbuf, ybuf, 1, sweeps) * 1e3, 3),
        note="one launch moving 68 KB: the time any single timed product pays before its bytes")
    del tiny

    # C1: Q8_0 2048 x 2048, one row; 64 copies (285 MB) rotate past the caches.
    n = k = 2048
    codes, sbits = synth.q8_0_matrix(synth.seed_for(0, 1), n, k)
    blocks = synth.q8_0_blocks(codes, sbits)
    copies = [hip.Dense.q8_0(n, k, blocks) for _ in range(64)]
    ms = timed_sweeps(H, stream, copies, xbuf, ybuf, 1, sweeps)
    b2b = back_to_back(H, stream, copies, xbuf, ybuf, 1, sweeps)
    algo = n * k * 34 // 32 + 4 * k + 4 * n
    out["c1_q8_0_gemv_2048x2048_b1"] = dict(avg_us=round(ms * 1e3, 3), bytes=algo, gb_s=gbs(algo, ms),
                                            frac=round(gbs(algo, ms) / HBM_PEAK_GBS, 4), copies=64,
                                            back_to_back_us=round(b2b * 1e3, 3),
                                            back_to_back_frac=round(gbs(algo, b2b) / HBM_PEAK_GBS, 4),
                                            above_floor_us=round((ms - floor_ms) * 1e3, 3))
    del copies

    # C3: ternary 4096 x 4096, rows 1 and 8; 64 copies (270 MB).
    n = k = 4096
    tcodes, tscales = synth.ternary_matrix(synth.seed_for(0, 3), n, k)
    copies = [hip.Dense.ternary(tcodes, tscales) for _ in range(64)]
    for b in (1, 8):
        ms = timed_sweeps(H, stream, copies, xbuf, ybuf, b, sweeps)
        b2b = back_to_back(H, stream, copies, xbuf, ybuf, b, sweeps)
        algo = n * k // 4 + n * 4 + b * (4 * k + 4 * n)
        out[f"c3_ternary_gemv_4096x4096_b{b}"] = dict(avg_us=round(ms * 1e3, 3), bytes=algo, gb_s=gbs(algo, ms),
                                                      frac=round(gbs(algo, ms) / HBM_PEAK_GBS, 4), copies=64,
                                                      back_to_back_us=round(b2b * 1e3, 3),
                                                      back_to_back_frac=round(gbs(algo, b2b) / HBM_PEAK_GBS, 4))
    del copies

    # C4: the Q4_K set of a 3B layer (K x N): qkv 3072 x 4096, o 3072 x 3072,
    # gate/up 3072 x 16384, down 8192 x 3072; 3 copies of the set (311 MB as
    # the Q8_0 codes the device runs by default). The layers are made with
    # TRIT_HIP_Q4K=1, so they also hold their super-blocks: each row count is
    # timed on the requantized codes (the default path, TRIT_HIP_Q4K=0 at the
    # call) and on the native product from the super-blocks.
    shapes = [(4096, 3072), (3072, 3072), (16384, 3072), (3072, 8192)]
    sets = []
    saved = os.environ.get("TRIT_HIP_Q4K")
    os.environ["TRIT_HIP_Q4K"] = "1"
    for rep in range(3):
        sets += [hip.Dense.q4_k(nn, kk, synth.q4_k_blocks(synth.seed_for(0, 40 + i), nn, kk))
                 for i, (nn, kk) in enumerate(shapes)]
    q4k = sum(nn * kk * 144 // 256 for nn, kk in shapes)
    dev = sum(nn * kk * 34 // 32 for nn, kk in shapes)
    for b in (1, 4):
        io = sum(b * (nn + kk) * 4 for nn, kk in shapes)
        set_ms = {}
        for native in ("0", "1"):
            os.environ["TRIT_HIP_Q4K"] = native
            set_ms[native] = timed_sweeps(H, stream, sets, xbuf, ybuf, b, sweeps) * len(shapes)
        ms = set_ms["0"]
        os.environ["TRIT_HIP_Q4K"] = "0"  # back to back on the default path
        b2b = back_to_back(H, stream, sets, xbuf, ybuf, b, sweeps) * len(shapes)
        out[f"c4_q4_k_set_b{b}"] = dict(set_us=round(ms * 1e3, 2), q4_k_bytes=q4k + io,
                                        back_to_back_set_us=round(b2b * 1e3, 2),
                                        back_to_back_frac=round(gbs(q4k + io, b2b) / HBM_PEAK_GBS, 4),
                                        gb_s_q4_k_bytes=gbs(q4k + io, ms),
                                        frac=round(gbs(q4k + io, ms) / HBM_PEAK_GBS, 4),
                                        device_bytes=dev + io, gb_s_device_bytes=gbs(dev + io, ms),
                                        note="held as Trit's requantized Q8_0 codes (34 B per 32 weights)",
                                        native=dict(set_us=round(set_ms["1"] * 1e3, 2),
                                                    gb_s_q4_k_bytes=gbs(q4k + io, set_ms["1"]),
                                                    frac=round(gbs(q4k + io, set_ms["1"]) / HBM_PEAK_GBS, 4),
                                                    note="gemv_q4k_kernel from the 144-byte super-blocks "
                                                         "(opt-in: TRIT_HIP_Q4K=1 at load); VALU-bound"))
    if saved is None:
        os.environ.pop("TRIT_HIP_Q4K", None)
    else:
        os.environ["TRIT_HIP_Q4K"] = saved
    del sets

    # C5: prefill contraction, 1564 rows (1500 encoder + 64 text), K 2048.
    m, k = 1564, 2048
    H.upload(xbuf, synth.activations(synth.seed_for(0, 5), m, k))
    fwd = hip.lib().trit_hip_layer_forward_device
    res = {}
    total_ops, total_gemm_ms, total_call_ms = 0, 0.0, 0.0
    for i, n in enumerate((2048, 6144, 2048)):
        codes, sbits = synth.q8_0_matrix(synth.seed_for(0, 50 + i), n, k)
        layer = hip.Dense.q8_0(n, k, synth.q8_0_blocks(codes, sbits))
        gemm_ms = timed_sweeps(H, stream, [layer], xbuf, ybuf, m, sweeps)
        a, b = H.event(), H.event()
        H.record(a, stream)
        for _ in range(sweeps):
            hip.check(fwd(layer.h, xbuf, m, 0, ybuf, stream))
        H.record(b, stream)
        call_ms = H.elapsed_ms(a, b) / sweeps
        ops = 2 * m * n * k
        total_ops += ops
        total_gemm_ms += gemm_ms
        total_call_ms += call_ms
        res[f"n{n}"] = dict(gemm_us=round(gemm_ms * 1e3, 2), call_us=round(call_ms * 1e3, 2),
                            tops=round(ops / (gemm_ms * 1e-3) / 1e12, 1))
    # The exact group chain costs three vector operations per (row, output,
    # 32-group): convert the i32 dot, scale product, FMA -- the bound of
    # this bit-exact GEMM is the vector ALUs, not the matrix cores.
    valu_ops = 3 * m * sum((2048, 6144, 2048)) * (k // 32)
    out["c5_prefill_gemm_1564x2048"] = dict(
        products=res, ops=total_ops, gemm_us=round(total_gemm_ms * 1e3, 2),
        call_us=round(total_call_ms * 1e3, 2), tops=round(total_ops / (total_gemm_ms * 1e-3) / 1e12, 1),
        mfma_frac=round(total_ops / (total_gemm_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4), peak_tops=INT8_PEAK_TOPS,
        valu_ops=valu_ops, valu_bound_us=round(valu_ops / (VALU_PEAK_TOPS * 1e12) * 1e6, 1),
        valu_frac=round(valu_ops / (total_gemm_ms * 1e-3) / (VALU_PEAK_TOPS * 1e12), 4),
        note="gemm_us: the MFMA kernels (event-stamped); call_us adds the activation quantization pass; "
             "valu_frac: the exact f32 group chain's vector operations against the vector ALU peak")

    # Beam decode: one Whisper large-v3 decoder layer's step for 5 beams --
    # the f16 products of 5 rows (self q/k/v/o and cross q/o 1280 x 1280,
    # fc1 5120 x 1280, fc2 1280 x 5120, biases) over 8 copies of the layer
    # (367 MB), and the self-attention of the 5 beams over 448 keys each.
    shapes = [(1280, 1280)] * 6 + [(5120, 1280), (1280, 5120)]
    host = [(synth.f16_bits((synth.activations(synth.seed_for(0, 60 + i), nn, kk) * 0.02).astype(np.float32)),
             synth.activations(synth.seed_for(0, 70 + i), 1, nn)[0]) for i, (nn, kk) in enumerate(shapes)]
    f16s = [hip.Dense.f16(wb, bias) for _ in range(8) for wb, bias in host]
    del host
    ms = timed_sweeps(H, stream, f16s, xbuf, ybuf, 5, sweeps)
    per_layer_ms = ms * len(shapes)
    wbytes = sum(nn * kk * 2 + nn * 4 for nn, kk in shapes) + sum(5 * (nn + kk) * 4 for nn, kk in shapes)
    del f16s
    beams, tk, d, heads = 5, 448, 1280, 20
    kvb = tk * d * 4
    kv = H.malloc(2 * beams * kvb)
    H.upload(kv, synth.activations(synth.seed_for(0, 80), 2 * beams * tk, d))
    steps_dev = hip.lib().trit_hip_attention_steps_device
    keys = (C.c_void_p * beams)(*[kv.value + b * kvb for b in range(beams)])
    values = (C.c_void_p * beams)(*[kv.value + (beams + b) * kvb for b in range(beams)])
    tks = (C.c_int * beams)(*([tk] * beams))
    a, b = H.event(), H.event()
    hip.check(steps_dev(xbuf, d, keys, values, tks, beams, d, heads, heads, ybuf, stream))
    H.record(a, stream)
    for _ in range(sweeps):
        hip.check(steps_dev(xbuf, d, keys, values, tks, beams, d, heads, heads, ybuf, stream))
    H.record(b, stream)
    att_ms = H.elapsed_ms(a, b) / sweeps
    H.L.hipFree(kv)
    att_bytes = 2 * beams * kvb
    out["beam_step_whisper_large_v3_5beams"] = dict(
        products_us=round(per_layer_ms * 1e3, 2), products_bytes=wbytes, products_gb_s=gbs(wbytes, per_layer_ms),
        products_frac=round(gbs(wbytes, per_layer_ms) / HBM_PEAK_GBS, 4),
        attention_us=round(att_ms * 1e3, 2), attention_bytes=att_bytes, attention_gb_s=gbs(att_bytes, att_ms),
        note="per decoder layer: eight f16 products of 5 rows (kernel time, event-stamped), and "
             "trit_hip_attention_steps_device over 448 f32 keys a beam (back-to-back calls, host launch included)")

    # The audio encoder before the decoder (Whisper large-v3's, as Voxtral
    # runs it): its stem and 4 of its 32 layers (d 1280, 20 heads, MLP 5120,
    # 128 mel bins, 1500 positions) with Q8_0 products; wall clock of
    # trit_hip_encoder_encode (host copies of the 3000 x 128 window and the
    # 1500 x 1280 output included), best of 5.
    ecfg = dict(d=1280, layers=4, heads=20, ffn=5120, mels=128, positions=1500)
    ed, eff = ecfg["d"], ecfg["ffn"]

    def eq8(n, k, i):
        codes, sbits = synth.q8_0_matrix(synth.seed_for(0, 90 + i), n, k, scale="normal", sigma=0.2)
        return hip.Dense.q8_0(n, k, synth.q8_0_blocks(codes, sbits), np.zeros(n, np.float32))

    shared = [eq8(3 * ed, ed, 0), eq8(ed, ed, 1), eq8(eff, ed, 2), eq8(ed, eff, 3)]
    norms = [np.ones(ed, np.float32), np.zeros(ed, np.float32)] * (2 * ecfg["layers"] + 1)
    enc = hip.Encoder(ecfg, eq8(ed, 3 * ecfg["mels"], 4), eq8(ed, 3 * ed, 5),
                      np.zeros((ecfg["positions"], ed), np.float32), shared * ecfg["layers"], norms)
    mel = synth.activations(synth.seed_for(0, 96), 2 * ecfg["positions"], ecfg["mels"])
    enc.encode(mel)  # warm-up
    t_enc = min(_timed(lambda: enc.encode(mel)) for _ in range(5))
    enc0 = hip.Encoder(dict(ecfg, layers=1), eq8(ed, 3 * ecfg["mels"], 4), eq8(ed, 3 * ed, 5),
                       np.zeros((ecfg["positions"], ed), np.float32), shared, norms[:6])
    enc0.encode(mel)
    t_one = min(_timed(lambda: enc0.encode(mel)) for _ in range(5))
    per_layer = (t_enc - t_one) / (ecfg["layers"] - 1)
    out["audio_encoder_whisper_large_v3"] = dict(
        encode_4_layers_ms=round(t_enc * 1e3, 2), per_layer_ms=round(per_layer * 1e3, 3),
        stem_and_one_layer_ms=round(t_one * 1e3, 2), full_32_layers_ms_estimate=round((t_one + 31 * per_layer) * 1e3, 1),
        note="Q8_0 products (int8 MFMA for the 1500-row products), Trit's exact attention over 1500 positions")
    del enc, enc0, shared

    # The Qwen3-ASR audio encoder over 30 s of audio (3000 mel frames: 30
    # chunks of 100, 390 rows, windows of 8 chunks): Qwen3-ASR's stem (128
    # mel bins, 480 channels; the 9-input first convolution in f32, the
    # others and conv_out Q8_0 on the matrix cores) under a d 1024, 16-head,
    # MLP 4096 stack with Q8_0 products, 8 layers timed against 1 (wall
    # clock of trit_hip_asr_encoder_encode, host copies included, best of 5).
    acfg = dict(d=1024, layers=8, heads=16, ffn=4096, mels=128, channels=480, chunk=100, window_chunks=8,
                out=2048, max_positions=1500)
    ad, aff, ach, frames = acfg["d"], acfg["ffn"], acfg["channels"], 3000
    c1 = synth.activations(synth.seed_for(0, 97), ach, 9) * np.float32(0.3)
    convs = [hip.Dense.f32(c1, np.zeros(ach, np.float32)), eq8(ach, 9 * ach, 6), eq8(ach, 9 * ach, 7)]
    conv_out = eq8(ad, ach * 16, 8)
    shared = [eq8(3 * ad, ad, 9), eq8(ad, ad, 10), eq8(aff, ad, 11), eq8(ad, aff, 12)]
    proj = [eq8(ad, ad, 13), eq8(acfg["out"], ad, 14)]
    norms = [np.ones(ad, np.float32), np.zeros(ad, np.float32)] * (2 * acfg["layers"] + 1)
    amel = synth.activations(synth.seed_for(0, 98), frames, acfg["mels"])
    asr = hip.AsrEncoder(acfg, convs, conv_out, shared * acfg["layers"], norms, *proj)
    asr.encode(amel, frames)  # warm-up
    t_asr = min(_timed(lambda: asr.encode(amel, frames)) for _ in range(5))
    asr1 = hip.AsrEncoder(dict(acfg, layers=1), convs, conv_out, shared, norms[:6], *proj)
    asr1.encode(amel, frames)
    t_asr1 = min(_timed(lambda: asr1.encode(amel, frames)) for _ in range(5))
    per = (t_asr - t_asr1) / (acfg["layers"] - 1)
    out["audio_encoder_qwen3_asr_30s"] = dict(
        rows=asr.rows(frames), encode_8_layers_ms=round(t_asr * 1e3, 2), per_layer_ms=round(per * 1e3, 3),
        stem_one_layer_and_projections_ms=round(t_asr1 * 1e3, 2),
        layers_24_ms_estimate=round((t_asr1 + 23 * per) * 1e3, 1),
        note="3000 mel frames; f32 first convolution, Q8_0 elsewhere (int8 MFMA for the many-row products, "
             "K tails included), Trit's exact attention within 104-row windows")
    del asr, asr1, shared, convs, conv_out, proj

    # C5 end to end: one decoder layer of the prefill's shape (hidden 2048,
    # 16/8 heads x 128, SwiGLU 3072) over the 1564-row prompt: the MFMA
    # products, q/k norm + rotary + cache append, causal GQA attention on
    # the matrix cores, and the (one-row) head of a 1024-token vocabulary.
    c5 = dict(d=2048, ffn=3072, layers=1, heads=16, kv_heads=8, head_dim=128, vocab=1024, eps=1e-6,
              rope_base=1e6, qk_norm=1)
    lm5 = model.build_decoder(synth.lm_weights(c5, config=5))
    p5 = synth.prompt(5, m, c5["vocab"])
    sess = lm5.session(m, 0)
    sess.prefill(p5, want_logits=False)  # warm-up
    times = []
    for _ in range(3):
        sess.reset()
        t0 = time.perf_counter()
        sess.prefill(p5, want_logits=False)
        times.append(time.perf_counter() - t0)
    t5 = min(times)
    att_ops = 2 * 2 * c5["heads"] * c5["head_dim"] * (m * (m + 1) // 2)
    out["c5_prefill_layer_1564"] = dict(
        layer_ms=round(t5 * 1e3, 3), rows_per_s=round(m / t5, 1), attention_ops=att_ops,
        note="one layer over 1564 rows, wall clock of the prefill call (host synchronisation included)")
    del sess, lm5
    if not decode:
        return out

    # The decode loops: a greedy run timed by events around the generate
    # call (the persistent step where the model fits it, else the per-kernel
    # loop, one graph replay a token), in Trit's sum orders with f16 caches.
    def loop_rate(cfg, seed, steps=64, prompt_len=256, lmx=None, kinds=("q8_0", "f16")):
        lmx = lmx or model.build_decoder(synth.lm_weights(cfg, config=seed))
        px = synth.prompt(seed, prompt_len, cfg["vocab"])
        sx = lmx.session(prompt_len + steps, 0)
        sx.prefill(px, want_logits=False)
        sx.generate(8)  # warm-up: the step's graph is captured
        sx.reset()
        sx.prefill(px, want_logits=False)
        ev_a, ev_b = H.event(), H.event()
        toks = np.empty(steps, np.int32)
        pers = C.c_int(0)
        n = hip.check(hip.lib().trit_hip_session_generate_timed(sx.h, steps, None, 0,
                                                                toks.ctypes.data_as(C.c_void_p), ev_a, ev_b,
                                                                C.byref(pers)))
        ms = H.elapsed_ms(ev_a, ev_b)
        roof = step_roofline(cfg, prompt_len, n, ms, bool(pers.value), "default", *kinds)
        del sx, lmx
        return dict(tok_s=round((n - 1) / (ms * 1e-3), 1), us_per_forward=roof["us_per_forward"],
                    bytes_per_forward=roof["bytes_per_forward"], gb_s=roof["achieved"], frac=roof["frac"],
                    persistent=bool(pers.value), tokens=[int(t) for t in toks[:n]])

    # S1-mini's own load (Qwen3-0.6B's shape at Trit's Auto precision: int8
    # linears, 128-group activations, a tied int8-storage table with f32
    # math) on the persistent step: the configuration of Trit's published
    # decode figure (about 15 ms a token on a 7950X3D).
    auto = synth.auto_weights(synth.lm_weights(dict(synth.QWEN3_06B), config=11, sigma=0.1, norm_jitter=0.2))
    line = loop_rate(dict(synth.QWEN3_06B), 1, steps=128, lmx=model.build_decoder_auto(auto), kinds=("int8", "q8"))
    out["decode_s1mini_auto_precision"] = dict(
        line, note="S1-mini's load: int8 linears (f32 scale per 128), tied int8-storage table (f32 scale per 32, "
                   "f32 math); 256-token prompt, 128 greedy steps on the persistent step, Trit's sums, f16 caches")
    # A cleanup call's length (src/cleanup.rs:154,296): a 900-token prompt
    # (system turn, control line and an 800-token part) and 256 steps, past
    # 512 positions (the step's keys in rounds of 512).
    line = loop_rate(dict(synth.QWEN3_06B), 1, steps=256, prompt_len=900, lmx=model.build_decoder_auto(auto),
                     kinds=("int8", "q8"))
    line.pop("tokens")
    out["decode_s1mini_cleanup_900_prompt_256_steps"] = dict(
        line, note="S1-mini's load, a 900-token prompt then 256 greedy steps on the persistent step (Trit's sums, "
                   "f16 caches; the attention over up to 1156 keys in rounds of 512)")
    del auto
    # An audio-LLM decode after its prompt (config 5's 1564 rows:
    # 1500 audio-encoder rows and 64 text tokens): Qwen3-0.6B's shape, Q8_0
    # linears, 64 greedy steps on the persistent step.
    line = loop_rate(dict(synth.QWEN3_06B), 1, steps=64, prompt_len=1564)
    line.pop("tokens")
    out["decode_audio_llm_1564_prompt_64_steps"] = dict(
        line, note="Qwen3-0.6B's shape, Q8_0 linears, tied f16 head; a 1564-row prompt then 64 greedy steps on "
                   "the persistent step (Trit's sums, f16 caches; 1565-1627 keys in rounds of 512)")

    cfg17 = dict(synth.QWEN3_06B, d=2048, ffn=6144)
    lm17 = model.build_decoder(synth.lm_weights(cfg17, config=17))
    out["decode_qwen3_1.7b_shape"] = dict(
        loop_rate(cfg17, 17, lmx=lm17), note="Qwen3-1.7B's shape (d 2048, ffn 6144, 28 layers), Q8_0 linears, tied "
                                             "f16 head; 256-token prompt, 64 greedy steps on the persistent step")
    out["decode_qwen3_1.7b_shape"].pop("tokens")
    prev = os.environ.get("TRIT_HIP_STEP")
    os.environ["TRIT_HIP_STEP"] = "0"
    try:
        out["decode_qwen3_1.7b_shape_per_kernel_loop"] = dict(
            loop_rate(cfg17, 17, lmx=lm17), note="the same model on the per-kernel loop (TRIT_HIP_STEP=0; graph "
                                                 "replay a token)")
        out["decode_qwen3_1.7b_shape_per_kernel_loop"].pop("tokens")
        del lm17
        out["decode_qwen3_0.6b_shape_per_kernel_loop"] = dict(
            loop_rate(dict(synth.QWEN3_06B), 1), note="the same loop on the 0.6B shape (TRIT_HIP_STEP=0)")
        out["decode_qwen3_0.6b_shape_per_kernel_loop"].pop("tokens")
    finally:
        if prev is None:
            del os.environ["TRIT_HIP_STEP"]
        else:
            os.environ["TRIT_HIP_STEP"] = prev
    return out


def step_roofline(cfg, prompt, steps, step_ms, persistent, mode, linears="q8_0", table="f16", counted=False):
    """The decode loop's kernel: the persistent step (one launch runs every
    step of a generate call) timed with HIP events around it. Algorithmic
    bytes per forward: every linear weight once (Q8_0: 34 B per 32; int8:
    132 B per 128), the head (f16: 2 B a value; int8 storage: 36 B per 32),
    the keys and values of the positions attended (f16, or f32 in the exact
    mode; the average over the timed tokens), the embedding row and the norm
    weights; one launch holds steps - 1 forwards. The per-kernel fallback is
    one graph replay a step."""
    d, ffn, hd, L = cfg["d"], cfg["ffn"], cfg["head_dim"], cfg["layers"]
    qkv = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    num, den = (34, 32) if linears == "q8_0" else (132, 128)
    weights = L * (qkv * d + d * cfg["heads"] * hd + 2 * ffn * d + d * ffn) * num // den
    head = cfg["vocab"] * d * 2 if table == "f16" else cfg["vocab"] * d * 36 // 32
    # Step i < steps - 1 forwards a token at position prompt + i over
    # prompt + i + 1 keys; the last step only makes the final choice.
    forwards = steps - 1
    mean_keys = prompt + (forwards - 1) / 2.0 + 1
    kv = int(L * cfg["kv_heads"] * hd * 2 * (4 if mode == "exact" else 2) * mean_keys)
    small = (d * 2 if table == "f16" else d * 36 // 32) + L * (2 * d + 2 * hd) * 4 + d * 4
    per_forward = weights + head + kv + small
    launches = 1 if persistent else steps
    per_launch = per_forward * forwards // launches
    avg_ms = step_ms / launches
    # The counters were read for the bench's own workload only (counted: the
    # metric's line, 256-token prompt and 128 steps, on the step).
    measured = counted and persistent and prompt == 256 and steps == 128
    traffic = (STEP_TRAFFIC_BYTES if mode == "default" else EXACT_TRAFFIC_BYTES if mode == "exact" else None) \
        if measured else None
    achieved = per_launch / (avg_ms * 1e-3) / 1e9
    return dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBS, 4),
                traffic=traffic * forwards if traffic else None,
                kernel=(f"step_kernel<4,8,12,2,8,{'false' if mode == 'tree' else 'true'},"
                        f"{0 if linears == 'q8_0' else 1},{0 if table == 'f16' else 1},false,"
                        f"{'true' if mode == 'exact' else 'false'}>: the persistent decode step "
                        f"({'tree sums' if mode == 'tree' else 'Trit sum orders'}, one-pass attention, "
                        f"{'f32' if mode == 'exact' else 'f16'} keys and values), {steps} "
                        "steps (choice, 28 layers, head) in one launch") if persistent
                       else "the per-kernel decode step (graph replay)",
                bytes_per_launch=per_launch, bytes_per_forward=per_forward, forwards=forwards,
                avg_us=round(avg_ms * 1e3, 3), us_per_forward=round(step_ms * 1e3 / forwards, 3),
                traffic_per_forward=traffic,
                launches=launches,
                timing="HIP events recorded on the library's stream before and after the step launch "
                       "(trit_hip_session_generate_timed); the launch includes the final choice-only step")


STAMP_PHASES = [  # (name, from stamp, to stamp); every block runs every phase
    ("x hand-over (after down)", 0, 1), ("RMSNorm (Trit's serial sum)", 1, 2),
    ("quantize (qkv input)", 2, 3), ("qkv rows and put (XCD-local)", 3, 4),
    ("attention: key and value loads issued", 4, 5), ("attention: qkv hand-over (XCD-local)", 5, 6),
    ("attention: q/k norm, rotary, append, values to LDS", 6, 7),
    ("attention: 1/16 of the keys scored and put (XCD-local)", 7, 25),
    ("attention: score hand-over", 25, 27), ("attention: max, exp", 27, 8),
    ("attention: softmax sum (serial)", 8, 9), ("attention: p.V (serial) and put", 9, 10),
    ("attention -> o hand-over", 10, 11),
    ("quantize (o input)", 11, 12), ("o rows and put", 12, 13),
    ("x hand-over (after o)", 13, 14), ("RMSNorm", 14, 15), ("quantize (gate_up input)", 15, 16),
    ("gate_up rows, SwiGLU, put", 16, 17), ("h hand-over", 17, 18),
    ("quantize (down input)", 18, 19), ("down rows and put", 19, 20),
    ("a layer", 0, 20)]
HEAD_PHASES = [("x hand-over (last layer's down)", None, 21), ("final RMSNorm", 21, 22), ("head passes", 22, 23),
               ("best of the block and put", 23, 24)]


def stamp_pass(w, prompt, steps, step=8, layer=10):
    """The persistent step's phases on the measurement build
    (TRIT_HIP_LIBRARY=trit_amd/lib/libtrit_hip_stamps.so): thread 0 of each
    block stamps fixed points of one (step, layer) of the launch; per phase,
    the mean over the blocks of the shader-clock interval, converted to
    microseconds by each block's shader/wall clock ratio over the layer.
    Stamp 10 (the attention's outputs put) is the putting wave's; the
    others are thread 0's. For the layout of one key/value head an XCD
    (step_layout 3), where every block runs every phase."""
    lib = hip.lib()
    lm, linears, embed = build_layers(w)
    sess = lm.session(len(prompt) + steps, 0)
    cfg = w.cfg
    blocks = 256

    def run(stamp_layer):
        hip.check(lib.trit_hip_step_stamps(step, stamp_layer))
        sess.reset()
        sess.prefill(prompt, want_logits=False)
        sess.generate(steps)
        assert sess.step_layout == 3, sess.step_layout
        wall = np.zeros((blocks, 32), np.uint64)
        clk = np.zeros((blocks, 32), np.uint64)
        hip.check(lib.trit_hip_step_stamps_read(wall.ctypes.data_as(C.c_void_p), clk.ctypes.data_as(C.c_void_p),
                                                blocks))
        return wall.astype(np.float64), clk.astype(np.float64)

    run(layer)  # warm-up
    wall, clk = run(layer)
    # Shader-clock ticks per microsecond, per block, over the layer (wall: 100 MHz).
    rate = (clk[:, 20] - clk[:, 0]) / ((wall[:, 20] - wall[:, 0]) / 100.0)
    rows = []
    for name, a, b in STAMP_PHASES:
        us = (clk[:, b] - clk[:, a]) / rate
        rows.append(dict(phase=name, us=round(float(np.mean(us)), 3)))
    hwall, hclk = run(cfg["layers"])
    hrate = np.median(rate)
    head = []
    for name, a, b in HEAD_PHASES:
        if a is None:
            continue
        us = (hclk[:, b] - hclk[:, a]) / hrate
        head.append(dict(phase=name, us=round(float(np.mean(us)), 3)))
    hip.check(lib.trit_hip_step_stamps(-1, -1))
    sess.free()
    lm.free()
    for layer_ in linears:
        layer_.free()
    embed.free()
    return dict(step=step, layer=layer, prompt=len(prompt), steps=steps, shader_mhz=round(float(np.median(rate)), 1),
                layer_phases=rows, head_phases=head)


def loop_pass(steps):
    """The per-kernel decode loop (no persistent step) of the Qwen3-0.6B and
    Qwen3-1.7B shapes: a 256-token prompt, then `steps` greedy steps, timed
    around the steps. Meant to run with TRIT_HIP_STEP=0 (and TRIT_HIP_GRAPH=0
    for a per-kernel profile: each kernel then launches on its own)."""
    H = Hip()
    out = {}
    for name, cfg, seed in (("qwen3_0.6b", dict(synth.QWEN3_06B), 1),
                            ("qwen3_1.7b", dict(synth.QWEN3_06B, d=2048, ffn=6144), 17)):
        lm = model.build_decoder(synth.lm_weights(cfg, config=seed))
        p = synth.prompt(seed, 256, cfg["vocab"])
        s = lm.session(256 + steps + 8, 0)
        s.prefill(p, want_logits=False)
        s.generate(4)
        s.reset()
        s.prefill(p, want_logits=False)
        a, b = H.event(), H.event()
        toks = np.empty(steps, np.int32)
        pers = C.c_int(0)
        n = hip.check(hip.lib().trit_hip_session_generate_timed(s.h, steps, None, 0, toks.ctypes.data_as(C.c_void_p),
                                                                a, b, C.byref(pers)))
        ms = H.elapsed_ms(a, b)
        out[name] = dict(steps=n, ms=round(ms, 3), us_per_forward=round(ms * 1e3 / max(n - 1, 1), 1),
                         persistent=bool(pers.value))
        print(f"[loop-pass] {name}: {out[name]}", file=sys.stderr, flush=True)
        del s, lm
    return out


def cpu_configs(configs, min_s=0.3):
    """The oracle (Trit's AVX-512 VNNI path, restated; the pinned team of
    cpu_baseline) on the same product shapes and seeds as config_lines:
    cpu_us per call (or per set) beside each GPU line, and the ratio. As on
    the GPU, C1 and C3 rotate 64 copies of the weights and C4 three copies
    of the set, so the weights come from DRAM rather than the CPU caches;
    each runs for at least min_s seconds. C5 times the three 1564-row
    products once each."""
    from oracle import oracle as O

    isa = O.isa_best()

    def timed(fns):
        for fn in fns:
            fn()  # warm
        n, t0 = 0, time.perf_counter()
        while True:
            for fn in fns:
                fn()
            n += len(fns)
            dt = time.perf_counter() - t0
            if dt >= min_s:
                return dt / n * 1e6

    def q8(codes, sbits):
        return O.Int8(codes, sbits.view(np.float16).astype(np.float32), 32, True, isa)

    def note(key, cpu_us, gpu_us, sample):
        if key in configs:
            configs[key].update(cpu_us=round(cpu_us, 1), gpu_vs_cpu=round(cpu_us / gpu_us, 1), cpu_sample=sample)

    x = synth.activations(synth.seed_for(0, 77), 64, 8192)
    key = "c1_q8_0_gemv_2048x2048_b1"
    if key in configs:
        codes, sbits = synth.q8_0_matrix(synth.seed_for(0, 1), 2048, 2048)
        Ls = [q8(codes, sbits) for _ in range(64)]
        note(key, timed([lambda L=L: L(x[:1, :2048]) for L in Ls]), configs[key]["avg_us"],
             "one row over 64 copies of the weights (285 MB), for 0.3 s")
        del Ls
    tcodes, tscales = synth.ternary_matrix(synth.seed_for(0, 3), 4096, 4096)
    Ts = [O.Ternary(tcodes, tscales, isa) for _ in range(64)]
    for b in (1, 8):
        key = f"c3_ternary_gemv_4096x4096_b{b}"
        if key in configs:
            note(key, timed([lambda T=T: T(x[:b, :4096]) for T in Ts]), configs[key]["avg_us"],
                 f"{b} rows over 64 copies of the weights, for 0.3 s")
    del Ts
    shapes = [(4096, 3072), (3072, 3072), (16384, 3072), (3072, 8192)]
    set4 = []
    for i, (nn, kk) in enumerate(shapes):
        c, sc = O.q8_0_quantize(O.q4_k_expand(synth.q4_k_blocks(synth.seed_for(0, 40 + i), nn, kk)))
        for _ in range(3):
            set4.append((O.Int8(c.reshape(nn, kk), sc.reshape(nn, kk // 32), 32, True, isa), kk))
    for b in (1, 4):
        key = f"c4_q4_k_set_b{b}"
        if key in configs:
            per_set = timed([lambda L=L, kk=kk: L(x[:b, :kk]) for L, kk in set4]) * len(shapes)
            note(key, per_set, configs[key]["set_us"],
                 f"the four products at {b} rows (Q4_K expanded and requantized as Trit does), "
                 f"three copies of the set, for 0.3 s")
    del set4
    key = "c5_prefill_gemm_1564x2048"
    if key in configs:
        xa = synth.activations(synth.seed_for(0, 5), 1564, 2048)
        total = 0.0
        for i, n in enumerate((2048, 6144, 2048)):
            c, sb = synth.q8_0_matrix(synth.seed_for(0, 50 + i), n, 2048)
            layer = q8(c, sb)
            layer(xa[:64])
            t0 = time.perf_counter()
            layer(xa)
            total += time.perf_counter() - t0
        note(key, total * 1e6, configs[key]["gemm_us"], "the three 1564-row products, once each")
    key = "decode_s1mini_auto_precision"
    if key in configs:
        # The oracle at Auto precision (int8 linears, the Q8 table) with the
        # device's f16-rounded caches: the same tokens expected, bit for bit.
        auto = synth.auto_weights(synth.lm_weights(dict(synth.QWEN3_06B), config=11, sigma=0.1, norm_jitter=0.2))
        ref = O.Lm(auto.cfg, auto.base, isa, kv_f16=True)
        for li, layer in enumerate(auto.linears):
            for which, (c, sc) in enumerate(layer):
                ref.set_linear_int8(li, which, c, sc)
        ref.set_table(0, O.TABLE_Q8, *auto.table)
        del auto
        steps = len(configs[key]["tokens"])
        logits = ref.forward(synth.prompt(1, 256, synth.QWEN3_06B["vocab"]))
        tokens, t0 = [], time.perf_counter()
        for i in range(steps):
            tok = O.argmax(logits)
            tokens.append(tok)
            if i + 1 < steps:
                logits = ref.forward(np.array([tok], np.int32))
        cpu_s = time.perf_counter() - t0
        del ref
        line = configs[key]
        line["cpu_tok_s"] = round((steps - 1) / cpu_s, 2)
        line["gpu_vs_cpu"] = round(line["tok_s"] / line["cpu_tok_s"], 1)
        line["tokens_identical"] = tokens == line["tokens"]
        line["distinct_tokens"] = len(set(tokens))
        line["cpu_sample"] = (f"the oracle at Auto precision (int8 VNNI products, the Q8 table in f32), f16-rounded "
                              f"caches, the same 256-token prompt, {steps} greedy steps once")


def cpu_model():
    """lscpu's model name, vendor, family and model (a hypervisor may shorten
    the name; the family and model still tell the core)."""
    import subprocess

    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            fields[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    name = fields.get("Model name", "unknown")
    return (f"{name} ({fields.get('Vendor ID', '?')} family {fields.get('CPU family', '?')} model "
            f"{fields.get('Model', '?')}, {fields.get('CPU(s)', '?')} CPUs)")


def cpu_fairness():
    """The baseline's sanity bound: a compute-bound int8 product (Trit's
    int8 layer, 1564 x 2048 x 2048, 128-groups) on the pinned team against
    the team's own vpdpbusd peak (register-resident chains). Trit's kernels
    reach about 90-95 % of theirs (oploop/LEDGER.md:1128-1137)."""
    from oracle import oracle as O

    if O.isa_best() != O.AVX512:
        return None
    peak = O.vnni_peak()
    codes = synth.ints(synth.seed_for(0, 60), (2048, 2048), -127, 127).astype(np.int8)
    scales = (0.001 + 0.01 * synth.uniform(synth.seed_for(0, 61), (2048, 16))).astype(np.float32)
    layer = O.Int8(codes, scales, 128, False, O.AVX512)
    x = synth.activations(synth.seed_for(0, 5), 1564, 2048)
    for _ in range(3):  # the team's clocks up
        layer(x)
    best = min(_timed(lambda: layer(x)) for _ in range(7))
    rate = 1564 * 2048 * 2048 / best
    return dict(peak_tmacs=round(peak / 1e12, 3), product_tmacs=round(rate / 1e12, 3),
                frac_of_peak=round(rate / peak, 3),
                shape="int8-128 product 1564 x 2048 x 2048 (least of 7, after 3 warm-up runs) against 24 "
                      "register-resident vpdpbusd chains a thread on the same team (best of 3)")


def _timed(fn):
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def load_times(w, prompt):
    """Seconds to a ready decoder of the workload's shape: from host layers
    (Q8_0 blocks and the f16 table as Trit holds them), from a GGUF file
    (read, split and uploaded), and from the device weight-cache file
    (uploaded without converting); with the file sizes and the time to read
    each file alone (its pages were just written, so reads come from the
    page cache). The decoders' logits for the prompt agree bit for bit."""
    import tempfile

    from trit_amd import gguf_writer as G

    def best(fn, n=3):
        return min(_timed(fn) for _ in range(n))

    def read_file(path):
        with open(path, "rb") as f:
            while f.read(64 << 20):
                pass

    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        gguf = os.path.join(tmp, "lm.gguf")
        cache = os.path.join(tmp, "weights.bin")
        G.write_decoder(gguf, w)
        held = []

        def from_layers():
            lm, linears, embed = build_layers(w)
            for L in linears:
                L.free()
            embed.free()
            held.append(lm)

        out["from_layers_s"] = round(best(from_layers), 3)
        out["from_gguf_s"] = round(best(lambda: held.append(hip.CausalLm.from_gguf(gguf))), 3)
        held[-1].save(cache)
        out["from_cache_s"] = round(best(lambda: held.append(hip.CausalLm.load(cache))), 3)
        out["gguf_bytes"] = os.path.getsize(gguf)
        out["cache_bytes"] = os.path.getsize(cache)
        out["read_gguf_s"] = round(best(lambda: read_file(gguf)), 3)
        out["read_cache_s"] = round(best(lambda: read_file(cache)), 3)
        logits = []
        for lm in (held[0], held[3], held[-1]):
            s = lm.session(len(prompt) + 1, hip.EXACT)
            logits.append(s.prefill(prompt))
            s.free()
        out["same_logits"] = bool(all(np.array_equal(logits[0].view(np.uint32), x.view(np.uint32))
                                      for x in logits[1:]))
        for lm in held:
            lm.free()
    out["note"] = ("seconds to a ready decoder (best of 3): host layers through trit_hip_layer_q8_0/f16 + "
                   "trit_hip_decoder_new; trit_hip_decoder_from_gguf; trit_hip_decoder_load of the file "
                   "trit_hip_decoder_save wrote; read_*: the file read alone")
    return out


def lively_check(cfg, prompt, steps):
    """Greedy tokens of the workload's model with livelier weights (scales
    N(0, 0.1)/127, norms 1 +- 0.2) on the persistent step, against the
    oracle with the device's f16-rounded caches."""
    from oracle import oracle as O

    w = synth.lm_weights(cfg, config=11, sigma=0.1, norm_jitter=0.2)
    lm = model.build_decoder(w)
    s = lm.session(len(prompt) + steps, 0)
    logits = s.prefill(prompt)
    got = [int(t) for t in s.generate(steps)]
    persistent = bool(s.persistent)
    s.free()
    lm.free()
    ref = O.Lm(cfg, w, O.isa_best(), kv_f16=True)
    want_logits = ref.forward(prompt)
    want, lg = [], want_logits
    for i in range(steps):
        want.append(O.argmax(lg))
        if i + 1 < steps:
            lg = ref.forward(np.array([want[-1]], np.int32))
    same_logits = bool(np.array_equal(np.asarray(logits, np.float32).view(np.uint32), want_logits.view(np.uint32)))
    return dict(tokens_identical=got == want, prompt_logits_identical=same_logits, distinct_tokens=len(set(got)),
                persistent=persistent, weights="Q8_0 scales N(0, 0.1)/127, norms 1 +- 0.2 (seed 11)")


def cpu_baseline(w, prompt, steps, rounds):
    """Trit's loop on the oracle (Trit's f32 caches): the prompt once, then
    `rounds` runs of the greedy steps from the same prompt caches (the
    caches cut back to the prompt between runs); least and median, as
    src/cpu/v2/bench.rs:42-54 reports a kernel."""
    from oracle import oracle as O

    threads = O.team_start(0, 0)
    isa = O.isa_best()
    ref = O.Lm(w.cfg, w, isa)
    ref.reset()
    t0 = time.perf_counter()
    logits0 = ref.forward(prompt)
    t_prefill = time.perf_counter() - t0
    times = []
    for _ in range(rounds):
        ref.truncate(len(prompt))
        logits = logits0
        tokens = []
        t0 = time.perf_counter()
        for i in range(steps):
            tok = O.argmax(logits)
            tokens.append(tok)
            if i + 1 < steps:
                logits = ref.forward(np.array([tok], np.int32))
        times.append(time.perf_counter() - t0)
    del ref
    return dict(tokens=tokens, t_prefill=t_prefill, t_least=min(times), t_median=float(np.median(times)),
                rounds=rounds, threads=threads, isa={0: "scalar", 1: "avx2", 2: "avx512-vnni"}[isa])


def timed_mode(lm, prompt, steps, warmup, flags, H):
    """The same workload in another session mode (a session of its own):
    warm-up runs, then the prompt and one timed generate call, timed as the
    headline line is."""
    sess = lm.session(len(prompt) + steps, flags)
    for _ in range(warmup):
        sess.reset()
        sess.prefill(prompt, want_logits=False)
        sess.generate(steps)
    sess.reset()
    sess.prefill(prompt, want_logits=False)
    ev_a, ev_b = H.event(), H.event()
    out_tokens = np.empty(steps, np.int32)
    persistent = C.c_int(0)
    t0 = time.perf_counter()
    n = hip.check(hip.lib().trit_hip_session_generate_timed(sess.h, steps, None, 0,
                                                            out_tokens.ctypes.data_as(C.c_void_p), ev_a, ev_b,
                                                            C.byref(persistent)))
    t = time.perf_counter() - t0
    step_ms = H.elapsed_ms(ev_a, ev_b)
    sess.free()
    forwards = max(n - 1, 1)
    return dict(value=round(forwards / t, 2), ms_per_step=round(t / forwards * 1e3, 4), step_ms=step_ms,
                persistent=bool(persistent.value), tokens=[int(x) for x in out_tokens[:n]],
                kv_cache="f32", sums="trit order (bit-exact: Trit's own arithmetic)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="greedy decode tokens timed")
    ap.add_argument("--warmup", type=int, default=1, help="untimed prefill + decode runs")
    ap.add_argument("--prompt", type=int, default=256)
    ap.add_argument("--mode", choices=["default", "exact", "tree"], default="default",
                    help="default: Trit's sums with f16 keys and values; exact: f32 keys and values; "
                         "tree: tree sums (not Trit's bits)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-product configuration lines")
    ap.add_argument("--sweeps", type=int, default=20, help="decode-order GEMV sweeps for the roofline")
    ap.add_argument("--cpu-rounds", type=int, default=5, help="timed runs of the CPU baseline's greedy steps")
    ap.add_argument("--configs-pass", action="store_true",
                    help="only the per-product configuration lines (for profiler runs)")
    ap.add_argument("--load-pass", action="store_true",
                    help="only the load times of the workload's decoder: from host layers, from a GGUF file, "
                         "from the device weight-cache file")
    ap.add_argument("--stamp-pass", action="store_true",
                    help="only the persistent step's phase stamps (needs the measurement build: "
                         "python -m trit_amd.build --stamps, then TRIT_HIP_LIBRARY=trit_amd/lib/libtrit_hip_stamps.so)")
    ap.add_argument("--products-pass", action="store_true",
                    help="only the per-product configurations (C1, C3, C4, C5 and the others before the decode "
                         "loops): no persistent-step launch, for rocprofv3")
    ap.add_argument("--loop-pass", action="store_true",
                    help="only the per-kernel decode loop of the 0.6B and 1.7B shapes (run it with TRIT_HIP_STEP=0 "
                         "TRIT_HIP_GRAPH=0 under rocprofv3 --kernel-trace --stats)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="only the roofline sweeps and a 256 MiB device copy (the counter scale for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "the token loop runs on one GPU: Trit's decoder has no multi-GPU path, "
                                   "so only --gpus 1 is measured", "n_gpus": args.gpus}))
        sys.exit(2)

    cfg = dict(synth.QWEN3_06B)
    t0 = time.perf_counter()
    w = synth.lm_weights(cfg, config=1)
    prompt = synth.prompt(1, args.prompt, cfg["vocab"])
    print(f"[bench] weights generated in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)

    hip.init(0)
    if args.configs_pass:
        print(json.dumps({"configs_pass": True, "configs": config_lines(Hip(), sweeps=args.sweeps)}), flush=True)
        return
    if args.load_pass:
        print(json.dumps({"load_pass": True, **load_times(w, prompt)}), flush=True)
        return
    if args.products_pass:
        print(json.dumps({"products_pass": True, "configs": config_lines(Hip(), sweeps=args.sweeps, decode=False)}),
              flush=True)
        return
    if args.loop_pass:
        print(json.dumps({"loop_pass": True, **loop_pass(args.steps)}), flush=True)
        return
    if args.stamp_pass:
        print(json.dumps({"stamp_pass": True, **stamp_pass(w, prompt, args.steps)}), flush=True)
        return
    lm, linears, embed = build_layers(w)
    if args.profile_pass:
        H = Hip()
        roof = gemv_roofline(H, linears, cfg, args.sweeps)
        copy_bytes = 256 << 20
        src, dst = H.malloc(copy_bytes), H.malloc(copy_bytes)
        H.ok(H.L.hipMemcpy(dst, src, C.c_size_t(copy_bytes), 3), "hipMemcpy")
        print(json.dumps({"profile_pass": True, "roofline": roof, "copy_bytes": copy_bytes}), flush=True)
        return
    flags = {"default": 0, "exact": hip.EXACT, "tree": hip.TREE_SUMS}[args.mode]
    max_pos = args.prompt + args.steps
    sess = lm.session(max_pos, flags)
    for _ in range(args.warmup):
        sess.reset()
        sess.prefill(prompt, want_logits=False)
        sess.generate(args.steps)
    print("[bench] warm-up done", file=sys.stderr, flush=True)

    sess.reset()
    print("[bench] timed prefill + decode ...", file=sys.stderr, flush=True)
    H = Hip()
    t0 = time.perf_counter()
    sess.prefill(prompt, want_logits=False)
    t_prefill = time.perf_counter() - t0
    ev_a, ev_b = H.event(), H.event()
    out_tokens = np.empty(args.steps, np.int32)
    persistent = C.c_int(0)
    t0 = time.perf_counter()
    n = hip.check(hip.lib().trit_hip_session_generate_timed(sess.h, args.steps, None, 0,
                                                            out_tokens.ctypes.data_as(C.c_void_p), ev_a, ev_b,
                                                            C.byref(persistent)))
    t_decode = time.perf_counter() - t0
    tokens = out_tokens[:n]
    step_ms = H.elapsed_ms(ev_a, ev_b)
    # Tokens per second as forwards per second: the first token is chosen
    # from the prompt's logits, and each later one costs one forward of the
    # token before it; `steps` tokens take steps - 1 forwards. (Trit's loop
    # also forwards the last token, whose logits nothing reads.)
    forwards = max(len(tokens) - 1, 1)
    value = forwards / t_decode
    print(f"[bench] gpu decode {value:.1f} tok/s (device {forwards / step_ms * 1e3:.1f}), "
          f"prefill {args.prompt / t_prefill:.1f} tok/s", file=sys.stderr, flush=True)
    step_roof = step_roofline(cfg, args.prompt, args.steps, step_ms, bool(persistent.value), args.mode, counted=True)
    exact = None
    if args.mode == "default":
        print("[bench] exact mode (f32 keys and values) ...", file=sys.stderr, flush=True)
        exact = timed_mode(lm, prompt, args.steps, args.warmup, hip.EXACT, H)
        exact["roofline"] = step_roofline(cfg, args.prompt, args.steps, exact.pop("step_ms"), exact["persistent"],
                                          "exact", counted=True)
        print(f"[bench] exact mode {exact['value']} tok/s", file=sys.stderr, flush=True)

    print("[bench] roofline sweep ...", file=sys.stderr, flush=True)
    roof = gemv_roofline(H, linears, cfg, args.sweeps)
    print(f"[bench] roofline {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}%)", file=sys.stderr, flush=True)

    configs = None
    if not args.no_configs:
        print("[bench] product configurations ...", file=sys.stderr, flush=True)
        configs = config_lines(H)
        print(f"[bench] configurations: {json.dumps(configs)}", file=sys.stderr, flush=True)

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(t_decode / forwards * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded splitmix64 counter-hash streams, Box-Muller normals; random-init weights "
                "of the named shape)",
        "config": {"workload": f"qwen3-0.6b-shape q8_0 decoder: {args.prompt}-token prefill then {args.steps} "
                               f"greedy decode steps ({forwards} forwards; tokens/s = forwards/s), batch 1, "
                               "tied f16 head", "layers": 28, "d": 1024, "heads": "16/8x128",
                   "ffn": 3072, "vocab": 151936, "prompt": args.prompt, "mode": args.mode,
                   "kv_cache": "f32" if args.mode == "exact" else "f16",
                   "sums": "tree" if args.mode == "tree" else "trit order (bit-exact)"},
        "prefill_tokens_per_s": round(args.prompt / t_prefill, 1),
        "roofline": step_roof,
        "gemv_roofline": roof,
    }
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cb = cpu_baseline(w, prompt, args.steps, args.cpu_rounds)
        cpu_forwards = max(args.steps - 1, 1)
        cpu_value = cpu_forwards / cb["t_least"]
        out["cpu_baseline"] = {
            "value": round(cpu_value, 2), "unit": "tokens/s", "cores": cb["threads"], "kind": "port",
            "median_value": round(cpu_forwards / cb["t_median"], 2), "cpu": cpu_model(),
            "sample": f"the same workload: {args.prompt}-token prefill once ({cb['t_prefill']:.2f} s), then "
                      f"{cb['rounds']} timed runs of the {args.steps} greedy steps from the prompt's caches "
                      f"(least {cb['t_least']:.2f} s, median {cb['t_median']:.2f} s; value from the least), "
                      f"{cb['isa']} path, one pinned thread per core of the largest L3 domain"}
        fair = cpu_fairness()
        if fair:
            out["cpu_baseline"]["fairness"] = fair
        out["tokens_identical"] = [int(t) for t in tokens] == cb["tokens"]
        if exact:
            exact["tokens_identical"] = exact.pop("tokens") == cb["tokens"]
            exact["gpu_vs_cpu"] = round(exact["value"] / cpu_value, 2)
        out["gpu_vs_cpu"] = round(value / cpu_value, 2)
        # The workload's weights settle on one repeated token, so the check
        # above cannot see a wrong step; the same model with livelier weights
        # gives a stream of different tokens, held against the f16-cache
        # oracle (the device's caches) bit for bit.
        print("[bench] lively-weights token check ...", file=sys.stderr, flush=True)
        out["lively_check"] = lively_check(cfg, prompt, args.steps)
        if configs:
            print("[bench] cpu configurations ...", file=sys.stderr, flush=True)
            cpu_configs(configs)
    if exact:
        exact.pop("tokens", None)
        out["exact_mode"] = exact
    if configs:
        for line in configs.values():
            line.pop("tokens", None)
        out["configs"] = configs
    print(json.dumps(out), flush=True)
    # Device memory is released before the interpreter exits.
    sess.free()
    lm.free()
    for layer in linears:
        layer.free()
    embed.free()


if __name__ == "__main__":
    main()
