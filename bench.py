#!/usr/bin/env python3
"""One-GPU benchmark of the gfx950 quantized matrix-product path.

Workload (the shape its metric is quoted on): the
Q8 FFN matmuls of one Qwen2.5-0.5B decode token through all 24 layers —
per layer the fused gate+up GEMV (2 x 4864 x 896, one launch, as the
reference fuses them: src/model.c:547-561) and the down GEMV (896 x 4864).
A step streams 24 distinct layers of weights (353 MB); two device copies of
the model alternate between steps (706 MB > the 256 MB Infinity Cache), so
every step reads its weights from HBM. Inputs are resident in HBM before the
timed region; each step replays one captured HIP graph of the 48 launches.

value = algorithmic bytes per step (weight blocks + int8 activations + f32
activation scales + f32 outputs) / measured step time, in GB/s.

Also reported: the roofline of the dominant kernel (the gate+up GEMV; average
launch duration from HIP events around back-to-back launches), the full
decode-token matmul set (q/k/v fused + o + gate/up + down for 24 layers plus
the LM head: 97 launches) as decode tok/s, the other BASELINE shapes, and the
reference's own AVX2 kernel (compiled from its sources, oracle/_ref) timed on
this host's cores on the same weights.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
smq = importlib.import_module("smolmoe-c99_amd")
synth = importlib.import_module("smolmoe-c99_amd.synth")

HBM_PEAK_GBS = 8000.0
DIM, HIDDEN, LAYERS, VOCAB = 896, 4864, 24, 151936
Q_DIM, KV_DIM = 896, 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def q8_bytes(rows, cols, ntok=1):
    """Algorithmic bytes of one Q8 matmul: weights + int8 x + f32 x scales + f32 outputs."""
    nb = (cols + 31) // 32
    return rows * nb * 36 + ntok * (nb * 32 + nb * 4) + ntok * rows * 4


class Act:
    """A quantized activation (ntok rows of `cols`) resident on the GPU."""

    def __init__(self, seed, ntok, cols):
        nb = (cols + 31) // 32
        x = synth.activations(seed, ntok, cols)
        self.x = smq.DeviceBuffer.from_array(x)
        self.d = smq.DeviceBuffer(ntok * nb * 4)
        self.q = smq.DeviceBuffer(ntok * nb * 32)
        smq.quantize_q8_rows(self.x, ntok, cols, self.d, self.q)


class Layer:
    def __init__(self, seed):
        self.host = {}
        self.dev = {}
        shapes = {"qkv": (Q_DIM + 2 * KV_DIM, DIM), "o": (DIM, Q_DIM), "gate": (HIDDEN, DIM), "up": (HIDDEN, DIM),
                  "down": (DIM, HIDDEN)}
        for k, (name, (rows, cols)) in enumerate(shapes.items()):
            w = synth.q8_weights(seed + k, rows, cols)
            self.host[name] = w
            self.dev[name] = (smq.DeviceBuffer.from_array(w), rows, cols)
        self.bias = smq.DeviceBuffer.from_array(synth.normal(seed + 9, Q_DIM + 2 * KV_DIM, 0.02))

    def copy(self):
        c = Layer.__new__(Layer)
        c.host = self.host
        c.dev = {}
        for name, (buf, rows, cols) in self.dev.items():
            nbuf = smq.DeviceBuffer(buf.nbytes)
            nbuf.copy_from(buf)
            c.dev[name] = (nbuf, rows, cols)
        c.bias = self.bias
        return c

    def qmat(self, name):
        buf, rows, cols = self.dev[name]
        return smq.QMat(buf, rows, cols)


def timed_graph(graphs, reps):
    """Milliseconds per replay of `graphs` (cycled), events around all replays."""
    smq.synchronize()
    smq.timer_start()
    for i in range(reps):
        graphs[i % len(graphs)].launch()
    return smq.timer_stop() / reps


def cpu_baseline(model, acts_x, acts_h, threads_list, budget_s, gpu_out):
    """The reference's AVX2 gemm (oracle/_ref, compiled from its kernels.c /
    kernels_x86.c) over the same FFN step: per layer the fused gate+up rows
    then the down rows, rows split statically over the threads (the caller is
    worker 0). Falls back to the oracle's scalar restatement ("port")."""
    import oracle
    orc = oracle.Oracle()
    if oracle.Reference.available():
        ref = oracle.Reference()
        fn, kind, name = ref.fn_addr("gemm_q8_avx2"), "reference", "gemm_q8_avx2 (reference kernels.c/kernels_x86.c)"
    else:
        fn, kind, name = orc.gemm_fn_addr(False), "port", "orc_gemm (oracle scalar restatement)"
    mats, rows, nbs, xds, xqs = [], [], [], [], []
    for l, layer in enumerate(model):
        gu = np.concatenate([layer.host["gate"], layer.host["up"]])
        mats += [np.ascontiguousarray(gu).reshape(-1), np.ascontiguousarray(layer.host["down"]).reshape(-1)]
        rows += [2 * HIDDEN, DIM]
        nbs += [DIM // 32, HIDDEN // 32]
        xds += [acts_x[l][0], acts_h[l][0]]
        xqs += [acts_x[l][1], acts_h[l][1]]
    gate = None
    if kind == "reference":
        # BASELINE parity gate: the CPU number counts only if the reference's
        # own kernel gives the GPU's bits on these inputs (layer 0, both matmuls).
        gate = True
        for m in range(2):
            want = ref.gemm(mats[m], nbs[m] * 36, xds[m], xqs[m], rows[m], 1, nbs[m], variant="avx2")
            gate = gate and np.array_equal(want.view(np.uint32), gpu_out[m].view(np.uint32))
    out = {}
    for threads in threads_list:
        one = orc.time_gemm_pass(fn, mats, rows, nbs, xds, xqs, 1, 36, threads, 1)
        reps = max(2, min(200, int(budget_s / max(one, 1e-4))))
        best = orc.time_gemm_pass(fn, mats, rows, nbs, xds, xqs, 1, 36, threads, reps)
        out[threads] = (best, reps)
    return kind, name, out, gate


def traffic_probe():
    """Short program for rocprofv3 --pmc runs: 8 launches of the dominant
    kernel (fused gate+up GEMV, 9728x896 Q8) on 8 distinct weight copies, then
    one 256 MiB device-to-device copy whose FETCH_SIZE / WRITE_SIZE calibrate the
    counters (expected 262,144 KiB each)."""
    smq.init(0)
    layer = Layer(1000)
    ax = Act(2000, 1, DIM)
    gu = smq.DeviceBuffer(2 * HIDDEN * 4)
    mats = []
    for _ in range(8):
        g_ = smq.DeviceBuffer(layer.dev["gate"][0].nbytes)
        u_ = smq.DeviceBuffer(layer.dev["up"][0].nbytes)
        g_.copy_from(layer.dev["gate"][0])
        u_.copy_from(layer.dev["up"][0])
        mats.append((smq.QMat(g_, HIDDEN, DIM), smq.QMat(u_, HIDDEN, DIM)))
    big = [smq.DeviceBuffer(256 << 20) for _ in range(2)]
    big[0].fill(1)
    smq.synchronize()
    for g_, u_ in mats:
        smq.matmul([(g_, None, gu.ptr), (u_, None, gu.ptr + HIDDEN * 4)], ax.d, ax.q, 1)
    smq.synchronize()
    big[1].copy_from(big[0])
    smq.synchronize()
    print("traffic probe done", flush=True)


def summarize_pmc(fetch_dir, write_dir):
    """Per-dispatch HBM traffic of the gate+up GEMV from two rocprofv3 --pmc
    runs of --traffic-probe, scaled by the copy's counter reading."""
    import csv
    import glob

    def read(d, counter):
        rows = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            rows += [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == counter]
        gemv = [float(r["Counter_Value"]) for r in rows if "k_gemv" in r["Kernel_Name"]]
        copy = sum(float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]
                   and float(r["Counter_Value"]) > 1e5)
        return gemv, copy

    fetch, fcopy = read(fetch_dir, "FETCH_SIZE")
    write, wcopy = read(write_dir, "WRITE_SIZE")
    expect = 256 * 1024.0  # KiB moved by the 256 MiB copy
    fscale, wscale = expect / fcopy, expect / wcopy
    f_kib = float(np.median(fetch)) * fscale
    w_kib = float(np.median(write)) * wscale
    out = {"fetch_kib_raw_median": float(np.median(fetch)), "write_kib_raw_median": float(np.median(write)),
           "copy_fetch_kib_raw": fcopy, "copy_write_kib_raw": wcopy, "fetch_scale": fscale, "write_scale": wscale,
           "traffic_bytes": int((f_kib + w_kib) * 1024), "algorithmic_bytes": q8_bytes(2 * HIDDEN, DIM),
           "dispatches": len(fetch)}
    print(json.dumps(out))
    return out


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--traffic-probe":
        traffic_probe()
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize-pmc":
        summarize_pmc(sys.argv[2], sys.argv[3])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=3.0, help="seconds of CPU timing per thread count")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    t_start = time.time()
    log("bench: init", smq.init(0), smq.kernels_select())
    t0 = time.time()
    model = [Layer(1000 + 16 * l) for l in range(LAYERS)]
    head_host = synth.q8_weights(1999, VOCAB, DIM)
    head = [smq.DeviceBuffer.from_array(head_host)]
    log(f"bench: generated and uploaded 24 layers + LM head in {time.time() - t0:.1f}s")
    copies = [model, [layer.copy() for layer in model]]
    head.append(smq.DeviceBuffer(head[0].nbytes))
    head[1].copy_from(head[0])

    # activations per layer: x (attention/FFN input, 896) and h (FFN hidden, 4864)
    ax = [Act(2000 + l, 1, DIM) for l in range(LAYERS)]
    ah = [Act(3000 + l, 1, HIDDEN) for l in range(LAYERS)]
    smq.numeric_check()
    gu_out = [smq.DeviceBuffer(2 * HIDDEN * 4) for _ in range(LAYERS)]
    y_out = [smq.DeviceBuffer(DIM * 4) for _ in range(LAYERS)]
    qkv_out = smq.DeviceBuffer((Q_DIM + 2 * KV_DIM) * 4)
    o_out = smq.DeviceBuffer(DIM * 4)
    logits = smq.DeviceBuffer(VOCAB * 4)

    def ffn_layer(layer, l, with_down=True):
        g_, u_ = layer.qmat("gate"), layer.qmat("up")
        smq.matmul([(g_, None, gu_out[l].ptr), (u_, None, gu_out[l].ptr + HIDDEN * 4)], ax[l].d, ax[l].q, 1)
        if with_down:
            smq.matmul([(layer.qmat("down"), None, y_out[l])], ah[l].d, ah[l].q, 1)

    def ffn_step(m):
        for l, layer in enumerate(m):
            ffn_layer(layer, l)

    def gateup_only(m):
        for l, layer in enumerate(m):
            ffn_layer(layer, l, with_down=False)

    def decode_matmuls(m, hd):
        for l, layer in enumerate(m):
            qkv = layer.qmat("qkv")
            smq.matmul([(qkv, layer.bias, qkv_out)], ax[l].d, ax[l].q, 1)
            smq.matmul([(layer.qmat("o"), None, o_out)], ax[l].d, ax[l].q, 1)
            ffn_layer(layer, l)
        smq.gemm_q8(hd, 28 * 36, ax[0].d, ax[0].q, VOCAB, 1, 28, logits, VOCAB)

    # one checked eager step (bounds checks on), then timing without host checks
    ffn_step(copies[0])
    smq.numeric_check()
    smq.set_checks(False)

    step_graphs = [smq.capture(lambda m=m: ffn_step(m)) for m in copies]
    step_bytes = LAYERS * (q8_bytes(2 * HIDDEN, DIM) + q8_bytes(DIM, HIDDEN))
    for i in range(args.warmup):
        step_graphs[i % 2].launch()
    ms_per_step = timed_graph(step_graphs, args.steps)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    smq.numeric_check()
    gpu_layer0 = [gu_out[0].download(np.float32), y_out[0].download(np.float32)]  # for the CPU parity gate
    log(f"bench: FFN step {ms_per_step * 1e3:.1f} us, {value:.0f} GB/s")

    # dominant kernel: gate+up GEMV (k_gemv<Q8, RT=8>), back-to-back launches
    gu_graphs = [smq.capture(lambda m=m: gateup_only(m)) for m in copies]
    timed_graph(gu_graphs, 4)
    reps = max(20, args.steps)
    gu_ms = timed_graph(gu_graphs, reps) / LAYERS
    gu_bytes = q8_bytes(2 * HIDDEN, DIM)
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    log(f"bench: gate+up GEMV {gu_ms * 1e3:.2f} us/launch, {gu_gbs:.0f} GB/s")

    extra = {}
    if not args.no_extra:
        dec_graphs = [smq.capture(lambda m=m, h=h: decode_matmuls(m, h)) for m, h in zip(copies, head)]
        timed_graph(dec_graphs, 4)
        dec_ms = timed_graph(dec_graphs, max(20, args.steps))
        dec_bytes = LAYERS * (q8_bytes(Q_DIM + 2 * KV_DIM, DIM) + q8_bytes(DIM, Q_DIM) + q8_bytes(2 * HIDDEN, DIM) +
                              q8_bytes(DIM, HIDDEN)) + q8_bytes(VOCAB, DIM)
        extra["decode_token_matmuls"] = {
            "what": "97 launches per token: 24 x (q/k/v fused+bias, o, gate+up fused, down) + LM head, Qwen2.5-0.5B",
            "us_per_token": round(dec_ms * 1e3, 2), "tok_s": round(1000.0 / dec_ms, 1),
            "GBps": round(dec_bytes / (dec_ms * 1e-3) / 1e9, 1)}
        log(f"bench: decode matmuls {dec_ms * 1e3:.1f} us/token = {1000 / dec_ms:.0f} tok/s")

        def single(name, fn, nbytes, per_graph, reps=10, note=None):
            """Per-launch time of fn(i), i = 0..per_graph-1 captured in one graph
            (fn picks distinct weight buffers by i), timed over `reps` replays."""
            gs = [smq.capture(lambda: [fn(i) for i in range(per_graph)] and None)]
            timed_graph(gs, 2)
            ms = timed_graph(gs, reps) / per_graph
            extra[name] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "pct_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
            if note:
                extra[name]["note"] = note
            log(f"bench: {name} {ms * 1e3:.2f} us {extra[name]['GBps']} GB/s")

        single("c3_lm_head_gemv_151936x896",
               lambda i: smq.gemm_q8(head[i % 2], 28 * 36, ax[0].d, ax[0].q, VOCAB, 1, 28, logits, VOCAB),
               q8_bytes(VOCAB, DIM), 16, note="2 copies of 153 MB alternated (306 MB > 256 MB Infinity Cache)")
        single("c1_down_gemv_896x4864",
               lambda i: smq.matmul([(copies[i // LAYERS % 2][i % LAYERS].qmat("down"), None, y_out[0])], ah[0].d,
                                    ah[0].q, 1),
               q8_bytes(DIM, HIDDEN), 2 * LAYERS, note="48 distinct 4.9 MB matrices in turn (235 MB)")
        # prefill: exact GEMM and int8-MFMA GEMM at batch 128 on the fused gate+up shape
        px = Act(4000, 128, DIM)
        pout = smq.DeviceBuffer(128 * 2 * HIDDEN * 4)

        def prefill(i):
            layer = copies[i // LAYERS % 2][i % LAYERS]
            smq.matmul([(layer.qmat("gate"), None, pout.ptr), (layer.qmat("up"), None, pout.ptr + 128 * HIDDEN * 4)],
                       px.d, px.q, 128)

        single("c1_prefill_exact_gemm_9728x896_b128", prefill, q8_bytes(2 * HIDDEN, DIM, 128), 8)
        smq.set_prefill_mfma(True)
        single("c1_prefill_mfma_gemm_9728x896_b128", prefill, q8_bytes(2 * HIDDEN, DIM, 128), 24)
        smq.set_prefill_mfma(False)
        ops = 2 * 2 * HIDDEN * DIM * 128
        for k in ("c1_prefill_exact_gemm_9728x896_b128", "c1_prefill_mfma_gemm_9728x896_b128"):
            e = extra[k]
            e["int_TOPS"] = round(ops / (e["us"] * 1e-6) / 1e12, 2)
            e["pct_int8_peak"] = round(100 * ops / (e["us"] * 1e-6) / 5.0e15, 2)
        qx = Act(5, 1, HIDDEN)
        single("quantize_q8_4864",
               lambda i: smq.quantize_q8_rows(qx.x, 1, HIDDEN, qx.d, qx.q), HIDDEN * 4 + HIDDEN + HIDDEN // 8, 32)

    cpu = None
    if not args.no_cpu:
        try:
            acts_x = [(synth_q(ax[l], DIM)) for l in range(LAYERS)]
            acts_h = [(synth_q(ah[l], HIDDEN)) for l in range(LAYERS)]
            ncpu = len(os.sched_getaffinity(0))
            threads = min(16, ncpu)
            kind, name, res, gate = cpu_baseline(copies[0], acts_x, acts_h, sorted({1, threads}), args.cpu_budget,
                                                 gpu_layer0)
            best, nreps = res[threads]
            cpu = {"value": round(step_bytes / best / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": kind,
                   "gpu_bit_identical_layer0": gate,
                   "sample": f"{name}: {nreps} passes over the same 24-layer FFN decode step (353 MB of Q8 weights, "
                             f"best pass {best * 1e3:.2f} ms); 1 thread: {step_bytes / res[1][0] / 1e9:.2f} GB/s; "
                             f"host {cpu_model()}, {ncpu} CPUs visible, rows split statically, caller is worker 0"}
            log(f"bench: cpu {cpu['value']} GB/s on {threads} threads ({kind})")
        except Exception as ex:  # the CPU leg must not hide the GPU result
            log(f"bench: cpu baseline failed: {ex!r}")

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "gemv_q8_gateup_9728x896_traffic.json")
    if os.path.exists(tfile):  # measured by two rocprofv3 --pmc runs of --traffic-probe (see that file)
        with open(tfile) as f:
            traffic = json.load(f).get("traffic_bytes")

    line = {
        "metric": "Q8_0/Q5_0 GEMV HBM GB/s (% of peak); decode tok/s at Qwen2.5-0.5B shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded N(0,0.02) weights packed by the q8pack rule, N(0,1) activations quantized on GPU",
        "config": {"workload": "configs[1]: Qwen2.5-0.5B Q8 FFN matmuls, batch 1 (decode GEMV), all 24 layers "
                               "(gate+up fused 9728x896 + down 896x4864 per layer), 353 MB/step, 2 model copies "
                               "alternated", "bytes_per_step": step_bytes, "parallelism": "none (1 GPU)"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "ffn_decode_tok_s": round(1000.0 / ms_per_step, 1),
        "roofline": {"kernel": "k_gemv<Q8,exact,RT=8,direct> (fused gate+up, 9728x896)", "bound": "hbm",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": gu_bytes, "us_per_launch": round(gu_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
        "wall_s": round(time.time() - t_start, 1),
    }
    print(json.dumps(line), flush=True)


def synth_q(act, cols):
    nb = (cols + 31) // 32
    return act.d.download(np.float32, nb), act.q.download(np.int8, nb * 32)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
