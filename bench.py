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
# HBM bytes per launch of the roofline kernel, from rocprofv3 --pmc runs of
# `bench.py --profile-pass` (profiles/gemv_row_q8_0_6144x1024_hbm_traffic.md):
# FETCH_SIZE 3313.1 KiB x 2.0 (the scale a 256 MiB device copy gives) plus
# WRITE_SIZE 48.0 KiB x 1.0.
GATE_UP_TRAFFIC_BYTES = round((3313.1 * 2.0 + 48.0) * 1024)


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
                kernel="gemv_row_kernel<4,1>: Q8_0 one-row product, the 6144x1024 gate_up weights",
                bytes_per_launch=algo, avg_us=round(avg_ms * 1e3, 3), launches=len(durations),
                timing="hipExtLaunchKernel start/stop events per launch, inside decode-order sweeps of "
                       "all 112 Q8_0 products (468 MB per sweep, past the 256 MB Infinity Cache)")


def cpu_baseline(w, prompt, steps):
    from oracle import oracle as O

    threads = O.team_start(0, 0)
    isa = O.isa_best()
    ref = O.Lm(w.cfg, w, isa)
    ref.reset()
    t0 = time.perf_counter()
    logits = ref.forward(prompt)
    t_prefill = time.perf_counter() - t0
    tokens = []
    t0 = time.perf_counter()
    for i in range(steps):
        tok = O.argmax(logits)
        tokens.append(tok)
        if i + 1 < steps:
            logits = ref.forward(np.array([tok], np.int32))
    t_decode = time.perf_counter() - t0
    del ref
    return dict(tokens=tokens, t_prefill=t_prefill, t_decode=t_decode, threads=threads,
                isa={0: "scalar", 1: "avx2", 2: "avx512-vnni"}[isa])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="greedy decode tokens timed")
    ap.add_argument("--warmup", type=int, default=1, help="untimed prefill + decode runs")
    ap.add_argument("--prompt", type=int, default=256)
    ap.add_argument("--mode", choices=["fast", "exact"], default="fast")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--sweeps", type=int, default=20, help="decode-order GEMV sweeps for the roofline")
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
    lm, linears, embed = build_layers(w)
    if args.profile_pass:
        H = Hip()
        roof = gemv_roofline(H, linears, cfg, args.sweeps)
        copy_bytes = 256 << 20
        src, dst = H.malloc(copy_bytes), H.malloc(copy_bytes)
        H.ok(H.L.hipMemcpy(dst, src, C.c_size_t(copy_bytes), 3), "hipMemcpy")
        print(json.dumps({"profile_pass": True, "roofline": roof, "copy_bytes": copy_bytes}), flush=True)
        return
    flags = hip.EXACT if args.mode == "exact" else 0
    max_pos = args.prompt + args.steps
    sess = lm.session(max_pos, flags)
    for _ in range(args.warmup):
        sess.reset()
        sess.prefill(prompt, want_logits=False)
        sess.generate(args.steps)
    print("[bench] warm-up done", file=sys.stderr, flush=True)

    sess.reset()
    print("[bench] timed prefill + decode ...", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    sess.prefill(prompt, want_logits=False)
    t_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    tokens = sess.generate(args.steps)
    t_decode = time.perf_counter() - t0
    value = len(tokens) / t_decode
    print(f"[bench] gpu decode {value:.1f} tok/s, prefill {args.prompt / t_prefill:.1f} tok/s",
          file=sys.stderr, flush=True)

    print("[bench] roofline sweep ...", file=sys.stderr, flush=True)
    H = Hip()
    roof = gemv_roofline(H, linears, cfg, args.sweeps)
    print(f"[bench] roofline {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}%)", file=sys.stderr, flush=True)

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(t_decode / max(len(tokens), 1) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded xorshift64* streams, random-init weights of the named shape)",
        "config": {"workload": "qwen3-0.6b-shape q8_0 decoder: 256-token prefill then 128 greedy decode steps, "
                               "batch 1, tied f16 head", "layers": 28, "d": 1024, "heads": "16/8x128",
                   "ffn": 3072, "vocab": 151936, "prompt": args.prompt, "mode": args.mode,
                   "kv_cache": "f32" if args.mode == "exact" else "f16"},
        "prefill_tokens_per_s": round(args.prompt / t_prefill, 1),
        "roofline": roof,
    }
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cb = cpu_baseline(w, prompt, args.steps)
        cpu_value = args.steps / cb["t_decode"]
        out["cpu_baseline"] = {
            "value": round(cpu_value, 2), "unit": "tokens/s", "cores": cb["threads"], "kind": "port",
            "sample": f"the same workload in full: {args.prompt}-token prefill ({cb['t_prefill']:.2f} s) then "
                      f"{args.steps} greedy steps ({cb['t_decode']:.2f} s), {cb['isa']} path"}
        out["tokens_identical"] = [int(t) for t in tokens] == cb["tokens"]
        out["gpu_vs_cpu"] = round(value / cpu_value, 2)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
