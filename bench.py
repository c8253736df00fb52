"""Benchmark of the fused-epilogue GEMM path on one MI355X.

Headline (`value`): FP32 fused GEMM 4096^3 with bias[N] + ReLU (BASELINE
config 2b), TFLOP/s over the timed steps (wall clock, inputs resident in
HBM).  One step = one `ta_run_ops` call of that fused op.  The same JSON
line carries, under "secondary", the decode SwiGLU MLP GEMVs (config 3,
HBM GB/s with weight copies rotated past the 256 MB last-level cache),
the batched GELU GEMM (config 2a), the deterministic split-K shapes
(config 4), the TinyLlama-shaped prefill GEMMs (config 5) and, for
reference only, the vendor library (hipBLASLt through torch.matmul) on the
headline and prefill shapes.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]

Synthetic inputs from numpy's PCG64 (seeded); no dataset or checkpoint.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tensor-ash_amd"))

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense FP32 matrix
PEAK_FP16_MFMA = 2516.6  # TFLOP/s, dense
PEAK_HBM = 8000.0  # GB/s
METRIC = "fused-GEMM TFLOP/s at 4096^3 f32 + decode-GEMV HBM GB/s (f16 W), 1 MI355X"
LLC_BYTES = 256 << 20


def roofline(bound: str, achieved: float, peak: float, unit: str, traffic=None, **extra) -> dict:
    """The roofline block of one measured kernel or step: `achieved` is
    algorithmic work (flops or bytes, each tensor once) per second."""
    out = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": traffic}
    out.update(extra)
    return out


def time_roofline(flops: float, nbytes: float, seconds: float, peak_tflops: float, traffic=None) -> dict:
    """Roofline of a shape that is compute- or bandwidth-bound depending on
    its balance: the bound is the larger of flops / peak and bytes / HBM
    peak; frac = that time / the measured time."""
    t_c, t_m = flops / (peak_tflops * 1e12), nbytes / (PEAK_HBM * 1e9)
    if t_c >= t_m:
        return roofline("mfma", flops / seconds / 1e12, peak_tflops, "TFLOP/s", traffic,
                        floor_us=round(t_c * 1e6, 3))
    return roofline("hbm", nbytes / seconds / 1e9, PEAK_HBM, "GB/s", traffic, floor_us=round(t_m * 1e6, 3))


def load_pmc_traffic() -> dict:
    """HBM bytes per launch of the secondary kernels, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE per dispatch, each
    scaled by the same counter on a plain copy): `key traffic_bytes=N`,
    per layer for the multi-layer decode launches (`layers=L`)."""
    out = {}
    try:
        for line in (ROOT / "profiles" / "secondary_pmc.txt").read_text().splitlines():
            parts = line.split()
            if len(parts) >= 2 and parts[1].startswith("traffic_bytes="):
                v = int(parts[1].split("=", 1)[1])
                # multi-layer decode launches: stored per layer
                for f in parts[2:]:
                    if f.startswith("layers="):
                        v //= int(f.split("=", 1)[1])
                out[parts[0]] = v
    except OSError:
        pass
    return out


PMC = {}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def median_ns(stats_list):
    return statistics.median([s.gpu_time_ns for s in stats_list])


def headline(ta, ex, steps: int, warmup: int, settle_ms: float):
    m = n = k = 4096
    rng = np.random.default_rng(31)
    ha = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    hb = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    hbias = rng.uniform(-1, 1, n).astype(np.float32)
    a, b = ex.tensor_from(ha), ex.tensor_from(hb)
    bias, c = ex.tensor_from(hbias), ex.tensor([m, n])
    op = ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_RELU))
    # Untimed clock settling (declared in the JSON line, not counted as
    # warm-up): a cold process needs ~20 ms of MFMA load before the chip
    # holds its steady clock.
    settled = 0.0
    t_settle = time.perf_counter()
    while settle_ms > 0 and (time.perf_counter() - t_settle) * 1e3 < settle_ms:
        ex.run_ops([op])
    settled = (time.perf_counter() - t_settle) * 1e3 if settle_ms > 0 else 0.0
    for _ in range(warmup):
        ex.run_ops([op])
    stats = []
    t0 = time.perf_counter()
    for _ in range(steps):
        stats.append(ex.run_ops([op]))
    wall = time.perf_counter() - t0
    flops = 2.0 * m * n * k
    kernel_ns = statistics.mean(s.gpu_time_ns for s in stats)
    # post-timing validation on 8 rows against float64 numpy
    got = ex.download(c)
    rows = rng.integers(0, m, 8)
    ref = np.maximum(ha[rows].astype(np.float64) @ hb.astype(np.float64) + hbias, 0.0)
    rel = float(np.max(np.abs(got[rows] - ref)) / np.max(np.abs(ref)))
    info = ex.dispatch_info_for(1, m, n, k)
    return dict(
        settle_ms=settled,
        wall_s=wall, ms_per_step=wall / steps * 1e3, value=flops / (wall / steps) / 1e12,
        kernel_ms=kernel_ns / 1e6, achieved=flops / kernel_ns / 1e3, kernel=info["kernel"],
        rel_err=rel, inputs=(ha, hb),
    )


def decode_mlp(ta, ex, rows_list=(1, 4, 8), iters=30, layers=16):
    """Config 3: h = silu(x@Wg) * (x@Wu); y = h@Wd + res, packed f16 weights.

    A decode forward runs its layers back to back (TinyLlama, whose MLP
    shape this is, has 22), so the step is timed the same way: one prepared
    op graph (hipGraph) chains `layers` MLP layers - 16, the most one
    decode-MLP launch holds (22 layers would be 66 ops, over the 64-op
    submission limit) - layer l reading the previous layer's y as x and as
    residual, over
    `copies` weight sets rotated so the working set exceeds the 256 MB
    last-level cache (every layer reads its weights from HBM).  step_us is
    the graph's GPU time / layers.  launch_us is one layer prepared alone,
    where the events also bracket the graph launch latency."""
    hdim, ffn = 2048, 5632
    w_bytes = 2 * (2 * hdim * ffn) + 2 * ffn * hdim
    copies = max(5, math.ceil(LLC_BYTES / w_bytes) + 1)
    rng = np.random.default_rng(41)
    weights = []
    for i in range(copies):
        ws = []
        for (kk, nn) in ((hdim, ffn), (hdim, ffn), (ffn, hdim)):
            w = (rng.standard_normal(kk * nn, dtype=np.float32) * 0.02).astype(np.float32)
            ws.append(ex.tensor_from(ta.pack_f16w_row_tiles(w, kk, nn, ta.f16w_row_tile_n(kk, nn)),
                                     shape=[kk, nn], f16=True))
        weights.append(ws)

    def layer_ops(x, y, up, h, w):
        wg, wu, wd = w
        return [ta.MatmulOp(x, wu, up, packed_b=True),
                ta.MatmulOp(x, wg, h, epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU,
                                                           binary=ta.BINARY_MUL, d=up), packed_b=True),
                ta.MatmulOp(h, wd, y, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0),
                            packed_b=True)]

    out = {}
    for m in rows_list:
        bufs = [ex.tensor_from(rng.uniform(-1, 1, (m, hdim)).astype(np.float32)) for _ in range(2)]
        up, h = ex.tensor([m, ffn]), ex.tensor([m, ffn])
        ops = []
        for l in range(layers):
            ops += layer_ops(bufs[l % 2], bufs[(l + 1) % 2], up, h, weights[l % copies])
        chain = ex.prepare_op_graph(ops)
        single = ex.prepare_op_graph(layer_ops(bufs[0], bufs[1], up, h, weights[0]))
        for _ in range(3):
            chain.run()
            single.run()
        stats = []
        t0 = time.perf_counter()
        for i in range(iters):
            stats.append(chain.run())
        wall = time.perf_counter() - t0
        single_ns = median_ns([single.run() for _ in range(iters)])
        bytes_step = w_bytes + 4 * m * (hdim + 2 * ffn + 2 * hdim)
        step_ns = median_ns(stats) / layers
        traffic = PMC.get(f"decode_M{m}")
        out[f"M{m}"] = dict(step_us=step_ns / 1e3, gbps=bytes_step / step_ns,
                            frac_hbm=bytes_step / step_ns / PEAK_HBM, bytes_per_step=bytes_step,
                            layers_per_graph=layers, launch_us=single_ns / 1e3,
                            wall_us_per_step=wall / iters / layers * 1e6,
                            roofline=roofline("hbm", bytes_step / step_ns, PEAK_HBM, "GB/s",
                                              traffic))
        chain.close()
        single.close()
    return out


def batched_gelu(ta, ex, iters=10):
    bt, m, n, k = 8, 2048, 2048, 2048
    rng = np.random.default_rng(21)
    a = ex.tensor_from(rng.standard_normal((bt, m, k), dtype=np.float32))
    b = ex.tensor_from((rng.standard_normal((k, n), dtype=np.float32) / math.sqrt(k)).astype(np.float32))
    bias = ex.tensor_from(rng.uniform(-1, 1, (bt, n)).astype(np.float32))
    c = ex.tensor([bt, m, n])
    op = ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_GELU))
    # ~25 ms of MFMA load first: the section follows memory-bound ones, and
    # the clock needs that long to settle.
    for _ in range(25):
        ex.run_ops([op])
    ns = median_ns([ex.run_ops([op]) for _ in range(iters)])
    flops = 2.0 * bt * m * n * k
    return dict(kernel_ms=ns / 1e6, tflops=flops / ns / 1e3, frac=flops / ns / 1e3 / PEAK_FP32_MFMA,
                kernel=ex.dispatch_info_for(bt, m, n, k)["kernel"],
                roofline=roofline("mfma", flops / ns / 1e3, PEAK_FP32_MFMA, "TFLOP/s",
                                  PMC.get("gelu_8x2048")))


def splitk(ta, ex, iters=10):
    out = {}
    rng = np.random.default_rng(51)
    for (m, n, k) in ((64, 256, 65536), (32, 128, 131072)):
        copies = 4
        As = [ex.tensor_from(rng.uniform(-1, 1, (m, k)).astype(np.float32)) for _ in range(copies)]
        Bs = [ex.tensor_from(rng.uniform(-1, 1, (k, n)).astype(np.float32)) for _ in range(copies)]
        c = ex.tensor([m, n])
        flops = 2.0 * m * n * k
        bytes_ = 4.0 * (m * k + k * n + m * n)
        for s in (8, 16, 32, 0):
            for i in range(copies):
                ex.run_matmuls_split_k2(As[i], Bs[i], c, s)
            ns = median_ns([ex.run_matmuls_split_k2(As[i % copies], Bs[i % copies], c, s)
                            for i in range(iters)])
            key = f"{m}x{n}x{k}_S{s if s else 'auto'}"
            out[key] = dict(us=ns / 1e3, tflops=flops / ns / 1e3, gbps=bytes_ / ns,
                            frac_mfma=flops / ns / 1e3 / PEAK_FP32_MFMA, frac_hbm=bytes_ / ns / PEAK_HBM,
                            roofline=time_roofline(flops, bytes_, ns * 1e-9, PEAK_FP32_MFMA,
                                                   PMC.get(f"splitk_{m}x{n}x{k}") if s == 0 else None))
    return out


def prefill_layer(ta, ex, iters=10):
    """Config 5 GEMMs (TinyLlama-1.1B-shaped, seq 512, f16 weights, f32 acts).
    Consecutive timed runs read different weight sets (`weight_copies` of
    them, together larger than the 256 MB last-level cache), as a prefill
    over all of a model's layers does."""
    s, hid, ffn, qkv = 512, 2048, 5632, 2560
    rng = np.random.default_rng(61)
    host_w = {}

    def wt(k, n, key):
        # Copies of one weight share their host values: only their number
        # (and so the bytes a rotation streams) matters to the caches.
        if key not in host_w:
            host_w[key] = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float32)
        return ex.tensor_from(host_w[key], f16=True)

    cold = lambda nbytes: max(3, math.ceil(LLC_BYTES / nbytes) + 1)  # sets whose sum exceeds the LLC
    x = ex.tensor_from(rng.uniform(-1, 1, (s, hid)).astype(np.float32))
    attn = ex.tensor_from(rng.uniform(-1, 1, (s, hid)).astype(np.float32))
    w_bytes = 2 * (hid * qkv + hid * hid + 2 * hid * ffn + ffn * hid)
    copies = cold(w_bytes)
    sets = [(wt(hid, qkv, "q"), wt(hid, hid, "o"), wt(hid, ffn, "g"), wt(hid, ffn, "u"), wt(ffn, hid, "d"))
            for _ in range(copies)]
    q, o, up, h, y = ex.tensor([s, qkv]), ex.tensor([s, hid]), ex.tensor([s, ffn]), ex.tensor([s, ffn]), ex.tensor([s, hid])

    def cases(ws):
        wq, wo, wg, wu, wd = ws
        return {
            "qkv_512x2560x2048": [ta.MatmulOp(x, wq, q)],
            "o_512x2048x2048": [ta.MatmulOp(attn, wo, o, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0))],
            "up_512x5632x2048": [ta.MatmulOp(x, wu, up)],
            "gate_silu_mul_512x5632x2048": [ta.MatmulOp(x, wg, h, epilogue=ta.Epilogue(activation=2, binary=2, d=up))],
            "down_512x2048x5632": [ta.MatmulOp(h, wd, y, epilogue=ta.Epilogue(binary=1, d=x, beta=1.0))],
        }

    per_set = [cases(ws) for ws in sets]

    def rotated(run, n_sets):
        for i in range(n_sets):
            run(i)
        return median_ns([run(i % n_sets) for i in range(max(iters, n_sets))])

    out = {"weight_copies": copies}
    total_ns = 0.0
    total_flops = 0.0
    total_bytes = 0.0
    case_w = {"qkv": ("q", hid, qkv, 0), "o": ("o", hid, hid, 1), "up": ("u", hid, ffn, 3),
              "gate": ("g", hid, ffn, 2), "down": ("d", ffn, hid, 4)}
    for name, ops in per_set[0].items():
        # A single GEMM alone: enough copies of its one weight to exceed the
        # LLC (the layer's sets alone would still fit).
        key, kk_w, nn_w, pos = case_w[name.split("_")[0]]
        n_case = cold(2 * kk_w * nn_w)
        extra = [wt(kk_w, nn_w, key) for _ in range(max(0, n_case - copies))]
        ws_case = [sets[i][pos] for i in range(copies)] + extra
        case_ops = [[ta.MatmulOp(op.a, w_i, op.c, epilogue=op.epilogue) for op in ops] for w_i in ws_case]
        ns = rotated(lambda i: ex.run_ops(case_ops[i]), len(case_ops))
        del case_ops, extra
        mm, nn, kk = [int(v) for v in name.split("_")[-1].split("x")]
        flops = 2.0 * mm * nn * kk
        # A f32, W f16, C f32 (+ D f32 for the binary epilogues)
        nbytes = 4.0 * mm * kk + 2.0 * kk * nn + 4.0 * mm * nn * (2 if ops[0].epilogue.binary else 1)
        out[name] = dict(us=ns / 1e3, tflops=flops / ns / 1e3,
                         kernel=ex.dispatch_info_for(1, mm, nn, kk, True)["kernel"],
                         roofline=time_roofline(flops, nbytes, ns * 1e-9, PEAK_FP16_MFMA,
                                                PMC.get(f"prefill_{name.split('_')[0]}")))
        total_ns += ns
        total_flops += flops
        total_bytes += nbytes
    out["layer_gemms"] = dict(us=total_ns / 1e3, tflops=total_flops / total_ns / 1e3,
                              note="sum of the five GEMMs, each its own ta_run_ops call",
                              roofline=time_roofline(total_flops, total_bytes, total_ns * 1e-9, PEAK_FP16_MFMA))
    # The layer as a prefill runs it: the five GEMMs in one dependent op
    # graph (one event pair).  up and gate run as one dual launch, which
    # also leaves the f16 copy of h that down reads; x and attn are
    # converted to f16 by one paired launch at the start, and x's copy
    # serves QKV and up/gate.
    layers = [[op for ops in c.values() for op in ops] for c in per_set]
    ns = rotated(lambda i: ex.run_op_graph(layers[i]), copies)
    out["layer_gemms_one_submission"] = dict(
        us=ns / 1e3, tflops=total_flops / ns / 1e3,
        roofline=time_roofline(total_flops, total_bytes, ns * 1e-9, PEAK_FP16_MFMA))
    # The same graph prepared once per weight set (prepare_op_graph:
    # captured as a hipGraph) and replayed, as a prefill that runs its
    # layers repeatedly would; the events bracket the replay.
    preps = [ex.prepare_op_graph(layer) for layer in layers]
    try:
        ns = rotated(lambda i: preps[i].run(), copies)
    finally:
        for prep in preps:
            prep.close()
    out["layer_gemms_prepared"] = dict(
        us=ns / 1e3, tflops=total_flops / ns / 1e3,
        roofline=time_roofline(total_flops, total_bytes, ns * 1e-9, PEAK_FP16_MFMA))
    return out


def gemv_chain(ta, ex, iters=30):
    """One TinyLlama decode step's seven GEMV jobs (q, k, v with normed-A;
    o with the residual; up and gate with normed-A and SiLU*up; down with
    the residual) as a GEMV chain: list-order launches (the default) and
    one persistent launch with grid barriers between dependent groups
    (ML_DEVICE_SCOPE=1).  Bytes = f16 weights plus the f32 activations read
    and written.  `packed_op_graph`: the same step with the weights packed
    in 64-column tiles (the decode layout) as one op graph: q, k and v share
    a launch, then o, then the normed MLP as one decode-MLP launch;
    `packed_prepared`: that graph captured once per weight set and
    replayed.  Consecutive timed steps read different weight sets
    (`copies` of them, together larger than the 256 MB last-level cache),
    as a decode over all of a model's layers does."""
    rng = np.random.default_rng(71)
    hid, ffn, kv = 2048, 5632, 256
    shapes = ((hid, hid), (hid, kv), (hid, kv), (hid, hid), (hid, ffn), (hid, ffn), (ffn, hid))
    nbytes = 2 * (2 * hid * hid + 2 * hid * kv + 2 * hid * ffn + ffn * hid)
    copies = max(3, math.ceil(LLC_BYTES / nbytes) + 1)
    x = ex.tensor_from(rng.uniform(-1, 1, (1, hid)).astype(np.float32))
    norm = ex.tensor_from(rng.uniform(0.5, 1.5, hid).astype(np.float32))
    q, k, v, o, up, g, y = (ex.tensor([1, n]) for n in (hid, kv, kv, hid, ffn, ffn, hid))
    E = ta.Epilogue
    nm = dict(normed_a=(norm, 1e-5))

    def step_ops(ws, **pb):
        wq, wk, wv, wo, wu, wg, wd = ws
        return [ta.MatmulOp(x, wq, q, **nm, **pb), ta.MatmulOp(x, wk, k, **nm, **pb),
                ta.MatmulOp(x, wv, v, **nm, **pb),
                ta.MatmulOp(q, wo, o, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0), **pb),
                ta.MatmulOp(o, wu, up, **nm, **pb),
                ta.MatmulOp(o, wg, g, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up),
                            **nm, **pb),
                ta.MatmulOp(g, wd, y, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=o, beta=1.0), **pb)]

    def rotated(run, n_sets):
        for i in range(2 * n_sets):
            run(i % n_sets)
        return median_ns([run(i % n_sets) for i in range(iters)])

    weights = lambda k_, n_: (rng.standard_normal(k_ * n_, dtype=np.float32) * 0.02).astype(np.float32)
    row_sets = [[ex.tensor_from(weights(kk, nn), shape=[kk, nn], f16=True) for kk, nn in shapes]
                for _ in range(copies)]
    chains = [step_ops(ws) for ws in row_sets]
    out = {"weight_bytes": nbytes, "weight_copies": copies}
    saved = os.environ.pop("ML_DEVICE_SCOPE", None)
    try:
        for name, env in (("list_order", None), ("persistent", "1")):
            if env:
                os.environ["ML_DEVICE_SCOPE"] = env
            else:
                os.environ.pop("ML_DEVICE_SCOPE", None)
            ns = rotated(lambda i: ex.run_gemv_chain(chains[i]), copies)
            out[name] = dict(us=ns / 1e3, gbps=nbytes / ns, frac_hbm=nbytes / ns / PEAK_HBM)
    finally:
        os.environ.pop("ML_DEVICE_SCOPE", None)
        if saved is not None:
            os.environ["ML_DEVICE_SCOPE"] = saved
    del chains, row_sets

    packed_sets = [[ex.tensor_from(ta.pack_f16w_row_tiles(weights(kk, nn), kk, nn, 64), shape=[kk, nn], f16=True)
                    for kk, nn in shapes] for _ in range(copies)]
    layers = [step_ops(ws, packed_b=True) for ws in packed_sets]
    ns = rotated(lambda i: ex.run_op_graph(layers[i]), copies)
    out["packed_op_graph"] = dict(us=ns / 1e3, gbps=nbytes / ns, frac_hbm=nbytes / ns / PEAK_HBM)
    preps = [ex.prepare_op_graph(layer) for layer in layers]
    try:
        ns = rotated(lambda i: preps[i].run(), copies)
    finally:
        for prep in preps:
            prep.close()
    out["packed_prepared"] = dict(us=ns / 1e3, gbps=nbytes / ns, frac_hbm=nbytes / ns / PEAK_HBM)
    return out


GEMV_CLASSES = (  # examples/bench_packed_gemv.rs:52-58 (label, N, K)
    ("kv_1x256x2048", 256, 2048),
    ("qo_1x2048x2048", 2048, 2048),
    ("up_1x5632x2048", 5632, 2048),
    ("down_1x2048x5632", 2048, 5632),
    ("lm_head_1x32000x2048", 32000, 2048),
)
REF_GEMV_FLOOR_FRAC = 0.80  # benchmarks/thesis-expectations.toml:27 (t2_min_bw_frac)


def decode_gemv_classes(ta, ex, iters=30):
    """The reference's decode GEMV classes (examples/bench_packed_gemv.rs:
    52-58) as standalone packed f16-weight launches at M = 1, one run_ops
    submission each (the HIP events bracket the launch).  `cold`: consecutive
    runs read different weight copies whose sum exceeds the 256 MB
    last-level cache, as a decode over all layers does; `warm`: the same
    weights every run, as the reference's example measures.  Bytes = f16
    W + f32 x + f32 y.  The reference's bar is each class at >= 0.80 of its
    bandwidth floor (benchmarks/thesis-expectations.toml:27)."""
    rng = np.random.default_rng(91)
    out = {}
    for name, n, k in GEMV_CLASSES:
        w_bytes = 2 * k * n
        copies = max(3, math.ceil(LLC_BYTES / w_bytes) + 1)
        w = (rng.standard_normal(k * n, dtype=np.float32) * 0.02).astype(np.float32)
        packed = ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n))
        ws = [ex.tensor_from(packed, shape=[k, n], f16=True) for _ in range(copies)]
        x = ex.tensor_from(rng.uniform(-1, 1, (1, k)).astype(np.float32))
        y = ex.tensor([1, n])
        ops = [ta.MatmulOp(x, wi, y, packed_b=True) for wi in ws]
        nbytes = w_bytes + 4 * (k + n)
        for i in range(2 * copies):
            ex.run_ops([ops[i % copies]])
        cold = median_ns([ex.run_ops([ops[i % copies]]) for i in range(max(iters, copies))])
        for _ in range(4):
            ex.run_ops([ops[0]])
        warm = median_ns([ex.run_ops([ops[0]]) for _ in range(iters)])
        entry = {"weight_copies": copies, "bytes": nbytes}
        for tag, ns in (("cold", cold), ("warm", warm)):
            frac = nbytes / ns / PEAK_HBM
            entry[tag] = dict(us=ns / 1e3, gbps=nbytes / ns, frac_hbm=frac,
                              meets_ref_floor=bool(frac >= REF_GEMV_FLOOR_FRAC),
                              roofline=roofline("hbm", nbytes / ns, PEAK_HBM, "GB/s",
                                                PMC.get(f"gemv_{name}") if tag == "cold" else None))
        out[name] = entry
        del ws, ops
    return out


def splitk_fused(ta, ex, iters=20):
    """Deep-K skinny f32 GEMMs with a fused epilogue: run_ops routes them
    through the deterministic split-K (the reduce applies the epilogue to
    the plane sum).  `data_parallel_us`: the same op forced onto one split."""
    rng = np.random.default_rng(53)
    out = {}
    for (m, n, k) in ((256, 256, 16384), (128, 512, 16384), (256, 1024, 8192)):
        a = ex.tensor_from(rng.uniform(-1, 1, (m, k)).astype(np.float32))
        b = ex.tensor_from(rng.uniform(-1, 1, (k, n)).astype(np.float32))
        bias = ex.tensor_from(rng.uniform(-1, 1, n).astype(np.float32))
        c = ex.tensor([m, n])
        op = ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_GELU))
        for _ in range(5):
            ex.run_ops([op])
        ns = median_ns([ex.run_ops([op]) for _ in range(iters)])
        dp = median_ns([ex.run_op_split_k2(op, 1) for _ in range(3)])
        flops = 2.0 * m * n * k
        bytes_ = 4.0 * (m * k + k * n + m * n + n)
        info = ex.dispatch_info_for(1, m, n, k)
        out[f"{m}x{n}x{k}_bias_gelu"] = dict(
            us=ns / 1e3, tflops=flops / ns / 1e3, splits=info["split_k2"], stage1=info["kernel"],
            data_parallel_us=dp / 1e3,
            roofline=time_roofline(flops, bytes_, ns * 1e-9, PEAK_FP32_MFMA,
                                   PMC.get(f"splitk_fused_{m}x{n}x{k}")))
    return out


TUNER_SHAPES = (  # (config, B, M, N, K, f16 weights); one shape per BASELINE config
    ("c1_512x512x512_f32", 1, 512, 512, 512, False),
    ("c2_4096x4096x4096_f32", 1, 4096, 4096, 4096, False),
    ("c3_gemv_1x5632x2048_f16w", 1, 1, 5632, 2048, True),
    ("c4_64x256x65536_f32", 1, 64, 256, 65536, False),
    ("c5_qkv_512x2560x2048_f16w", 1, 512, 2560, 2048, True),
)


def tuner(ta, ctx, iters=10):
    """The ML_TUNE measured auto-tuner (src/executor/tuning.rs:76-250) on
    one shape per BASELINE config, from an empty store: its pick (kernel and
    split count) and, beside it, every registry kernel that supports the
    shape forced through the executor's kernel selection (median of `iters`
    run_ops GPU times), plus the split counts of the split-K probe.  Run
    under rocprofv3 --pmc, the same dispatches give each candidate's
    counters (MFMA busy cycles, HBM bytes), which is what justifies a pick."""
    import shutil
    import tempfile
    # A private, empty tune store for the whole section (the store is read
    # when the executor is created and rewritten after every tuned shape).
    saved = os.environ.get("XDG_CACHE_HOME")
    store = tempfile.mkdtemp(prefix="ta_tune_")
    os.environ["XDG_CACHE_HOME"] = store
    try:
        return _tuner_runs(ta, ctx, iters)
    finally:
        if saved is None:
            os.environ.pop("XDG_CACHE_HOME", None)
        else:
            os.environ["XDG_CACHE_HOME"] = saved
        shutil.rmtree(store, ignore_errors=True)


def _tuner_runs(ta, ctx, iters):
    tune_ex = ta.Executor(ctx, tune=True)
    forced = {}
    rng = np.random.default_rng(81)
    out = {}
    for name, bt, m, n, k, f16 in TUNER_SHAPES:
        a = tune_ex.tensor_from(rng.uniform(-1, 1, (m, k)).astype(np.float32))
        b = tune_ex.tensor_from(rng.uniform(-1, 1, (k, n)).astype(np.float32), f16=f16)
        c = tune_ex.tensor([m, n])
        op = ta.MatmulOp(a, b, c)
        log(f"  tuner {name} ...")
        tune_ex.run_ops([op])  # tunes on first sight, then runs the pick
        pick = tune_ex.dispatch_info_for(bt, m, n, k, f16)
        picked_ns = median_ns([tune_ex.run_ops([op]) for _ in range(iters)])
        cands = {}
        for kname in ta.kernel_names():
            if kname not in forced:
                forced[kname] = ta.Executor(ctx, kernel_selection=kname, tune=False)
            fx = forced[kname]
            try:
                for _ in range(2):
                    fx.run_ops([op])
            except ta.TensorAshError:
                continue
            cands[kname] = median_ns([fx.run_ops([op]) for _ in range(iters)]) / 1e3
        entry = dict(pick=pick, pick_us=picked_ns / 1e3, candidates_us=cands)
        if not f16:
            splits = {}
            for sk in (4, 8, 16, 32, 64, 128):
                if k // sk < 128:
                    continue
                try:
                    tune_ex.run_matmuls_split_k2(a, b, c, sk)
                except ta.TensorAshError:
                    continue
                splits[sk] = median_ns([tune_ex.run_matmuls_split_k2(a, b, c, sk)
                                        for _ in range(iters)]) / 1e3
            entry["split_k2_us"] = splits
        out[name] = entry
    for fx in forced.values():
        fx.close()
    tune_ex.close()
    return out


def concurrency(ta, ex, iters=20):
    """Independent ops in one ta_run_ops call may run concurrently on
    several streams; the same ops as a dependent op graph run back to back
    on one.  Cases: TinyLlama decode Q/K/V projections (three packed f16
    GEMVs, M = 1), four independent 512x1024x2048 f16w GEMMs, and four
    long underfilled f32 GEMMs with a fused bias + GELU (256x256x16384,
    16 tiles each; the epilogue rules out split-K)."""
    rng = np.random.default_rng(91)

    def packed(k, n):
        w = (rng.standard_normal(k * n, dtype=np.float32) * 0.02).astype(np.float32)
        return ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)), shape=[k, n], f16=True)

    x = ex.tensor_from(rng.uniform(-1, 1, (1, 2048)).astype(np.float32))
    qkv = [ta.MatmulOp(x, packed(2048, n), ex.tensor([1, n]), packed_b=True) for n in (2048, 256, 256)]
    a = ex.tensor_from(rng.uniform(-1, 1, (512, 2048)).astype(np.float32))
    gemms = [ta.MatmulOp(a, ex.tensor_from((rng.standard_normal((2048, 1024), dtype=np.float32) * 0.02),
                                           f16=True), ex.tensor([512, 1024])) for _ in range(4)]
    bias = ex.tensor_from(rng.uniform(-1, 1, 256).astype(np.float32))
    big = [ta.MatmulOp(ex.tensor_from(rng.uniform(-1, 1, (256, 16384)).astype(np.float32)),
                       ex.tensor_from(rng.uniform(-1, 1, (16384, 256)).astype(np.float32)),
                       ex.tensor([256, 256]), epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_GELU))
           for _ in range(4)]
    out = {"note": "run_ops spreads independent ops over 4 streams only when the work beyond the "
                   "longest op is well above the ~40 us fork/join cost; one_lane_us forces one stream "
                   "(same routes); op_graph_us runs the same ops as a dependent graph"}
    def serial_run_ops(ops):
        os.environ["TA_RUN_OPS_LANES"] = "1"
        try:
            return ex.run_ops(ops)
        finally:
            del os.environ["TA_RUN_OPS_LANES"]

    for name, ops in (("decode_qkv_gemv_m1", qkv), ("four_512x1024x2048_f16w", gemms),
                      ("four_256x256x16384_f32_bias_gelu", big)):
        for _ in range(3):
            ex.run_ops(ops)
            serial_run_ops(ops)
            ex.run_op_graph(ops)
        auto = median_ns([ex.run_ops(ops) for _ in range(iters)])
        serial = median_ns([serial_run_ops(ops) for _ in range(iters)])
        graph = median_ns([ex.run_op_graph(ops) for _ in range(iters)])
        out[name] = dict(run_ops_us=auto / 1e3, one_lane_us=serial / 1e3, speedup=serial / auto,
                         op_graph_us=graph / 1e3)
    return out


ATTN_CASES = (  # name, H, H_kv, T, dh
    ("tinyllama_prefill_t512_dh64", 32, 4, 512, 64),
    ("llama_prefill_t2048_dh128", 32, 8, 2048, 128),
)


def causal_attn_flops(heads, t, dh):
    """Score and PV products over the causal triangle: 4 * dh flops per
    (query, attended key) pair, sum_i (i + 1) pairs per head."""
    return 4.0 * heads * dh * (t * (t + 1) / 2)


def attention(ta, ex, iters=10):
    """Causal prefill attention (run_flash_attention), f32 q/out, f32 and
    f16 caches, fresh prefill (kv_len = T)."""
    rng = np.random.default_rng(71)
    out = {}
    for name, heads, kvh, t, dh in ATTN_CASES:
        q = ex.tensor_from(rng.uniform(-1, 1, (heads, t, dh)).astype(np.float32))
        for kv16 in (False, True):
            kt = ex.tensor_from(rng.uniform(-1, 1, (kvh, dh, t)).astype(np.float32), f16=kv16)
            v = ex.tensor_from(rng.uniform(-1, 1, (kvh, t, dh)).astype(np.float32), f16=kv16)
            o = ex.tensor([heads, t, dh])
            desc = ta.FlashAttentionDesc(t, 0, float(1.0 / np.sqrt(dh)))
            for _ in range(3):
                ex.flash_attention(q, kt, v, o, desc)
            ns = median_ns([ex.flash_attention(q, kt, v, o, desc) for _ in range(iters)])
            out[name + ("_kv16" if kv16 else "_f32")] = dict(
                us=ns / 1e3, tflops=causal_attn_flops(heads, t, dh) / ns / 1e3)
    return out


# (name, kv_heads, group, dh, t_max, kv_len): TinyLlama-1.1B and Llama-3-8B
# decode steps.
DECODE_ATTN_CASES = [("tinyllama_kv640", 4, 8, 64, 2048, 640),
                     ("tinyllama_kv2048", 4, 8, 64, 2048, 2048),
                     ("llama3_8b_kv4096", 8, 4, 128, 8192, 4096)]


def token_loop(ta, ex, iters=20):
    """The GPU token loop ops: split-K decode attention (f32 and f16
    caches; bytes = the valid K and V prefix plus q and out), greedy argmax
    over a vocabulary, and the embedding gather of one token row."""
    rng = np.random.default_rng(81)
    out = {}
    for name, kvh, group, dh, t_max, kv_len in DECODE_ATTN_CASES:
        q = ex.tensor_from(rng.uniform(-1, 1, (kvh, group, dh)).astype(np.float32))
        scratch = ex.tensor([kvh * ta.ATTN_DECODE_MAX_CHUNKS * group * (dh + 2)])
        o = ex.tensor([kvh, group, dh])
        for kv16 in (False, True):
            kt = ex.tensor_from(rng.uniform(-1, 1, (kvh, dh, t_max)).astype(np.float32), f16=kv16)
            v = ex.tensor_from(rng.uniform(-1, 1, (kvh, t_max, dh)).astype(np.float32), f16=kv16)
            desc = ta.AttnDecodeDesc(kv_len, float(1.0 / np.sqrt(dh)))
            for _ in range(3):
                ex.attn_decode(q, kt, v, scratch, o, desc)
            ns = median_ns([ex.attn_decode(q, kt, v, scratch, o, desc) for _ in range(iters)])
            nbytes = 2 * kvh * kv_len * dh * (2 if kv16 else 4) + 2 * kvh * group * dh * 4
            out["attn_decode_" + name + ("_kv16" if kv16 else "_f32")] = dict(
                us=ns / 1e3, gbps=nbytes / ns, frac_hbm=nbytes / ns / PEAK_HBM)
    cell = ex.create_host_u32_buffer()
    for vocab in (32000, 128256):
        logits = ex.tensor_from(rng.uniform(-1, 1, vocab).astype(np.float32))
        for _ in range(3):
            ex.argmax(logits, cell)
        ns = median_ns([ex.argmax(logits, cell) for _ in range(iters)])
        out[f"argmax_{vocab}"] = dict(us=ns / 1e3, gbps=vocab * 4 / ns)
    table = ex.tensor_from(rng.uniform(-1, 1, (32000, 2048)).astype(np.float32), f16=True)
    row = ex.tensor([1, 2048])
    cell.set(12345)
    for _ in range(3):
        ex.embed_gather(cell, table, row)
    ns = median_ns([ex.embed_gather(cell, table, row) for _ in range(iters)])
    out["embed_gather_2048_f16"] = dict(us=ns / 1e3)
    return out


def vendor_reference(iters=20):
    """The vendor libraries on the same shapes, for reference only (not part
    of the product path; the role of the reference's
    benchmarks/cublas_bench/cublas_bench.cu): FP32 SGEMM from the
    hipBLASLt timing binary (HIP events, full FP32 compute type); f16 GEMM
    (torch's matmul, hipBLASLt on ROCm) and causal SDPA from torch, timed
    with torch events on torch's stream.  The f16 rows are f16 x f16 -> f16,
    the semantics of this build's a16 route, not of its f16w route (f32
    activations)."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return statistics.median(ts)

    out = {"library": "hipBLASLt FP32 via lib/vendor_bench (fastest of 8 heuristic candidates); "
                      "f16 GEMM and causal SDPA via torch " + torch.__version__}
    out.update(vendor_sgemm())
    g = torch.Generator(device="cuda").manual_seed(61)
    for (m, n, k) in ((512, 2560, 2048), (512, 2048, 2048), (512, 5632, 2048), (512, 2048, 5632)):
        x = torch.rand(m, k, device="cuda", generator=g, dtype=torch.float16) * 2 - 1
        w = torch.randn(k, n, device="cuda", generator=g, dtype=torch.float16) * 0.02
        us = timed(lambda: x @ w)
        out[f"hgemm_{m}x{n}x{k}_f16"] = dict(us=us, tflops=2.0 * m * n * k / us / 1e6)
    for name, heads, kvh, t, dh in ATTN_CASES:
        q = torch.rand(1, heads, t, dh, device="cuda", generator=g) * 2 - 1
        k = (torch.rand(1, kvh, t, dh, device="cuda", generator=g) * 2 - 1).repeat_interleave(heads // kvh, 1)
        v = (torch.rand(1, kvh, t, dh, device="cuda", generator=g) * 2 - 1).repeat_interleave(heads // kvh, 1)
        us = timed(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True))
        out[f"sdpa_causal_{name}_f32"] = dict(us=us, tflops=causal_attn_flops(heads, t, dh) / us / 1e6)
    torch.cuda.empty_cache()
    return out


def vendor_sgemm():
    """FP32 SGEMM of hipBLASLt on the BASELINE shapes (vendor_bench/cases.csv),
    run as a child process; median-based TFLOP/s."""
    import csv
    import io
    import subprocess
    pkg = Path(__file__).resolve().parent / "tensor-ash_amd"
    exe = pkg / "lib" / "vendor_bench"
    if not exe.exists():
        return {"sgemm_error": f"{exe} not built"}
    cases = (pkg / "vendor_bench" / "cases.csv").read_text()
    proc = subprocess.run([str(exe), "--iters", "20", "--warmup", "30"], input=cases, text=True,
                          capture_output=True, timeout=240)
    if proc.returncode != 0:
        return {"sgemm_error": proc.stderr.strip()[-400:]}
    out = {}
    for row in csv.DictReader(io.StringIO(proc.stdout)):
        out["sgemm_" + row["label"] + "_f32"] = dict(us=float(row["median_ms"]) * 1e3, tflops=float(row["tflops"]))
    return out


def cpu_baseline(inputs, target_s: float = 12.0):
    """The oracle's cpu_bmm (restatement of tools/test-support cpu_bmm:
    naive i-j-k, f64 accumulate) on host cores, over a bounded sample of
    output rows of the same 4096^3 problem."""
    import oracle
    ha, hb = inputs
    m, k = ha.shape
    n = hb.shape[1]
    # The GPU box gives one GPU a 16-thread CPU share (OMP_NUM_THREADS=16
    # there); the host may show more logical CPUs.
    threads = max(1, min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16") or 16), 16))
    a = np.ascontiguousarray(ha).reshape(-1)
    b = np.ascontiguousarray(hb).reshape(-1)
    out = np.zeros(m * n, np.float32)
    rows = threads
    t0 = time.perf_counter()
    oracle.cpu_bmm_rows(a, b, 1, m, n, k, 1.0, out, 0, rows, threads, reference_order=True)
    dt = time.perf_counter() - t0
    if dt < target_s / 4:
        more = int(rows * (target_s - dt) / max(dt, 1e-3))
        more = max(threads, min(more - more % threads, m - rows))
        t1 = time.perf_counter()
        oracle.cpu_bmm_rows(a, b, 1, m, n, k, 1.0, out, rows, rows + more, threads, reference_order=True)
        dt += time.perf_counter() - t1
        rows += more
    flops = 2.0 * rows * n * k
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                cpu_model=model, host_logical_cpus=os.cpu_count(),
                cores_note="threads capped at the one-GPU CPU share (16) of the GPU box",
                sample=f"cpu_bmm (f64-accumulate i-j-k oracle) on {rows} of 4096 output rows of the "
                       f"4096^3 GEMM, {dt:.1f} s on {threads} threads, extrapolation-free rate")


def load_traffic():
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, each scaled by the
    same counter on a plain copy of known size), or None."""
    p = ROOT / "profiles" / "gemm_f32_m256n256_4096cube_pmc.txt"
    try:
        for line in p.read_text().splitlines():
            if line.startswith("traffic_bytes="):
                return int(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10, help="untimed steps after clock settling")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--no-headline", action="store_true",
                    help="skip the headline (profiling runs of single sections)")
    ap.add_argument("--clock-settle-ms", type=float, default=50.0,
                    help="untimed headline GEMMs before warm-up until this many ms passed "
                         "(declared in the JSON line as clock_settle_ms)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy (rocprof counter calibration)")
    ap.add_argument("--sections", default="decode,gemv_classes,gemv_chain,gelu,splitk,splitk_fused,prefill,concurrency,attention,token_loop,vendor",
                    help="comma list of secondary sections to run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is not built", file=sys.stderr)
        return 2
    sections = set() if args.only_headline else set(args.sections.split(","))
    if args.calibrate_copy or "vendor" in sections:
        # torch's ROCm wheel carries its own HIP runtime; the runtime loaded
        # first serves the process, and torch only works on its own, so
        # torch is imported before libtensor_ash loads.
        import torch  # noqa: F401
    if args.calibrate_copy:
        # A plain copy kernel of known size: FETCH_SIZE / WRITE_SIZE of this
        # dispatch calibrate the counters used for the headline's traffic.
        import torch
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes_each_way": src.numel() * 4}), flush=True)
        return 0
    import tensor_ash as ta

    PMC.update(load_pmc_traffic())
    ctx = ta.Context()
    ex = ta.Executor(ctx, tune=False)
    hl = None
    if not args.no_headline:
        log("headline 4096^3 f32 fused GEMM ...")
        hl = headline(ta, ex, args.steps, args.warmup, args.clock_settle_ms)
    secondary = {}
    if "decode" in sections:
        log("decode SwiGLU MLP ...")
        secondary["decode_swiglu_mlp_f16w"] = decode_mlp(ta, ex)
    if "gemv_chain" in sections:
        log("decode GEMV chain ...")
        secondary["decode_gemv_chain_tinyllama"] = gemv_chain(ta, ex)
    if "gemv_classes" in sections:
        log("decode GEMV classes ...")
        secondary["decode_gemv_classes_m1"] = decode_gemv_classes(ta, ex)
    if "splitk_fused" in sections:
        log("split-K with fused epilogues ...")
        secondary["splitk_fused_epilogue_f32"] = splitk_fused(ta, ex)
    if "tuner" in sections:
        log("ML_TUNE candidates ...")
        secondary["tuner"] = tuner(ta, ctx)
    if "gelu" in sections:
        log("batched GELU GEMM ...")
        secondary["batched_gelu_8x2048^3"] = batched_gelu(ta, ex)
    if "splitk" in sections:
        log("split-K ...")
        secondary["splitk_f32"] = splitk(ta, ex)
    if "prefill" in sections:
        log("prefill layer GEMMs ...")
        secondary["prefill_tinyllama_m512_f16w"] = prefill_layer(ta, ex)
    if "concurrency" in sections:
        log("independent ops in one submission ...")
        secondary["run_ops_concurrency"] = concurrency(ta, ex)
    if "attention" in sections:
        log("causal prefill attention ...")
        secondary["causal_prefill_attention"] = attention(ta, ex)
    if "token_loop" in sections:
        log("token loop (decode attention, argmax, gather) ...")
        secondary["token_loop"] = token_loop(ta, ex)
    if "vendor" in sections:
        log("vendor library reference ...")
        secondary["vendor_reference"] = vendor_reference()
    if hl is None:
        print(json.dumps({"secondary": secondary}), flush=True)
        return 0
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(hl["inputs"])
    flops = 2.0 * 4096 ** 3
    line = {
        "metric": METRIC,
        "value": round(hl["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(hl["ms_per_step"], 4),
        "clock_settle_ms": round(hl["settle_ms"], 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy PCG64 uniform[-1,1]; inputs resident in HBM)",
        "config": {"workload": "gemm_f32_4096x4096x4096_bias_relu (BASELINE config 2b)",
                   "kernel": hl["kernel"], "m": 4096, "n": 4096, "k": 4096,
                   "epilogue": "bias[N]+relu", "validation_rel_err": hl["rel_err"]},
        "roofline": {"bound": "mfma", "achieved": round(hl["achieved"], 3), "peak": PEAK_FP32_MFMA,
                     "unit": "TFLOP/s", "frac": round(hl["achieved"] / PEAK_FP32_MFMA, 4),
                     "traffic": load_traffic(), "kernel_ms": round(hl["kernel_ms"], 4),
                     "flops_per_launch": flops},
        "cpu_baseline": cpu,
    }
    # The metric's second half (decode SwiGLU GEMVs, f16 W, HBM GB/s) at the
    # top level, beside the f32 headline.
    dec = secondary.get("decode_swiglu_mlp_f16w", {}).get("M1")
    if dec:
        line["decode_m1"] = {"workload": "decode SwiGLU MLP M=1 gate/up 2048x5632 + down 5632x2048 "
                                         "+ residual, f16 W packed (BASELINE config 3), 16 layers per launch",
                             "gbps": round(dec["gbps"], 1), "frac": round(dec["frac_hbm"], 4),
                             "step_us": round(dec["step_us"], 3), "roofline": dec["roofline"]}
    line["secondary"] = secondary
    # Short summary last, so a reader of the line's tail sees both halves.
    line["summary"] = {"gemm_4096_tflops": line["value"], "gemm_frac": line["roofline"]["frac"],
                       "decode_m1_gbps": line.get("decode_m1", {}).get("gbps"),
                       "decode_m1_frac": line.get("decode_m1", {}).get("frac")}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
