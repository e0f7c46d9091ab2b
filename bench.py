#!/usr/bin/env python3
"""One-GPU benchmark of the gfx950 quantized matrix-product path.

Workload (the shape its metric is quoted on): the
Q8 FFN matmuls of one Qwen2.5-0.5B decode token through all 24 layers —
per layer the gate and up GEMVs (4864 x 896) and the down GEMV (896 x 4864),
each with its layer's own quantized activation. A step streams 24 distinct
layers of weights (353 MB) as two grouped launches of the persistent
decode GEMV (48 gate/up GEMVs, then 24 down GEMVs: smq_gemv_grouped); two
device copies of the model alternate between steps (706 MB > the 256 MB
Infinity Cache), so every step reads its weights from HBM. Inputs are resident
in HBM before the timed region; the K timed steps are one captured HIP graph
(one graph launch per step is reported beside it). The same step as 48
launches in layer order (what a decode token must do, each layer waiting for
the previous one) is reported too.

value = algorithmic bytes per step (weight blocks + int8 activations + f32
activation scales + f32 outputs) / measured step time, in GB/s.

Also reported: the roofline of the dominant kernel (the gate+up GEMV; average
launch duration from HIP events around back-to-back launches), the full
decode-token matmul set (q/k/v fused + o + gate/up + down for 24 layers plus
the LM head: 97 launches) as decode tok/s, the other BASELINE shapes, the
reference's own AVX2 kernel (compiled from its sources, oracle/_ref) timed on
this host's cores on the same weights, and configs[4]: the whole random-init
Qwen2.5-0.5B-shaped decoder through the device-resident forward (prefill 512
ids, then 128 greedy decode steps as graph replays) with the reference's own
model_forward on the same checkpoint as CPU rate and bit-exactness gate.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --forward-only [--checkpoint PATH] [--decode-steps N] [--runs R]   (configs[4]
                                alone, for profiling; PATH from python bench.py --write-checkpoint PATH)
       python bench.py --anchor   (the HBM read/copy anchor and the hand-off anchor alone)
       python bench.py --q5-only   (configs[2] alone, for profiling)
       python bench.py --prefill-only   (the batched prefill GEMMs alone, for profiling)
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
FORWARD_RUNS = 10  # configs[4] runs on the GPU (median reported)
CPU_FORWARD_RUNS = 10  # configs[4] runs of the reference's model layer on the host (median reported)
HEAD_SAMPLES = 11  # timings of the headline graph and of the dominant kernel's graph; the median is reported
DIM, HIDDEN, LAYERS, VOCAB = 896, 4864, 24, 151936
Q_DIM, KV_DIM = 896, 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def q8_bytes(rows, cols, ntok=1, block=36):
    """Algorithmic bytes of one matmul (Q8 blocks of 36 B, Q5 of 22 B): weights + int8 x + f32 x scales
    + f32 outputs."""
    nb = (cols + 31) // 32
    return rows * nb * block + ntok * (nb * 32 + nb * 4) + ntok * rows * 4


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


SINGLE_SAMPLES = 11  # samples per single() shape: median reported, best beside it


def single_timing(extra, name, fn, nbytes, per_graph, reps=2, note=None):
    """Per-launch time of fn(i), i = 0..per_graph-1 captured in one graph (fn picks distinct weight
    buffers by i): SINGLE_SAMPLES timings of `reps` replays each; `us` is the median, `best_us` the best."""
    gs = [smq.capture(lambda: [fn(i) for i in range(per_graph)] and None)]
    timed_graph(gs, 2)
    med, best, _ = timed_samples(gs, reps, SINGLE_SAMPLES)
    ms, bms = med / per_graph, best / per_graph
    extra[name] = {"us": round(ms * 1e3, 2), "best_us": round(bms * 1e3, 2),
                   "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                   "pct_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                   "timing": f"median of {SINGLE_SAMPLES} samples of {reps} graph replays x {per_graph} launches"}
    if note:
        extra[name]["note"] = note
    log(f"bench: {name} {ms * 1e3:.2f} us (best {bms * 1e3:.2f}) {extra[name]['GBps']} GB/s")


def timed_samples(graphs, reps, samples):
    """`samples` independent timings of timed_graph(graphs, reps): (median, best, all) in ms per replay."""
    t = [timed_graph(graphs, reps) for _ in range(samples)]
    return float(np.median(t)), float(min(t)), t


def physical_cores():
    """(physical cores, logical CPUs) among the CPUs this process may run on: distinct
    (package, core) pairs of the affinity set, from sysfs."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
        except OSError:
            return None, len(cpus)
        cores.add((pkg, core))
    return len(cores), len(cpus)


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
        one, _ = orc.time_gemm_pass(fn, mats, rows, nbs, xds, xqs, 1, 36, threads, 1)
        reps = max(10, min(200, int(budget_s / max(one, 1e-4))))
        best, med = orc.time_gemm_pass(fn, mats, rows, nbs, xds, xqs, 1, 36, threads, reps)
        out[threads] = (best, reps, med)
    return kind, name, out, gate


def ffn_items(m, ax, ah, gu, yo):
    """The FFN step's 72 GEMVs (48 gate/up 4864x896, 24 down 896x4864), each with its layer's activation."""
    return ([(layer.qmat(k), None, gu[l].ptr + (HIDDEN * 4 if k == "up" else 0), False, ax[l].d, ax[l].q)
             for l, layer in enumerate(m) for k in ("gate", "up")] +
            [(layer.qmat("down"), None, yo[l], False, ah[l].d, ah[l].q) for l, layer in enumerate(m)])


def traffic_probe():
    """Short program for rocprofv3 --pmc runs: 4 launches of the dominant
    kernel (the planned FFN step: 72 GEMVs, 354 MB) alternating two model
    copies, then one 256 MiB device-to-device copy whose FETCH_SIZE /
    WRITE_SIZE calibrate the counters (expected 262,144 KiB each)."""
    smq.init(0)
    model = [Layer(1000 + 16 * l) for l in range(LAYERS)]
    copies = [model, [layer.copy() for layer in model]]
    ax = [Act(2000 + l, 1, DIM) for l in range(LAYERS)]
    ah = [Act(3000 + l, 1, HIDDEN) for l in range(LAYERS)]
    gu = [smq.DeviceBuffer(2 * HIDDEN * 4) for _ in range(LAYERS)]
    yo = [smq.DeviceBuffer(DIM * 4) for _ in range(LAYERS)]
    plans = [smq.GemvPlan(ffn_items(m, ax, ah, gu, yo)) for m in copies]
    big = [smq.DeviceBuffer(256 << 20) for _ in range(2)]
    big[0].fill(1)
    smq.synchronize()
    for i in range(4):
        plans[i % 2].launch()
    smq.synchronize()
    big[1].copy_from(big[0])
    smq.synchronize()
    print("traffic probe done", flush=True)


def summarize_pmc(fetch_dir, write_dir):
    """Per-dispatch HBM traffic of the planned FFN-step launch from two
    rocprofv3 --pmc runs of --traffic-probe, scaled by the copy's counter
    reading."""
    import csv
    import glob

    def read(d, counter):
        rows = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            rows += [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == counter]
        gemv = [float(r["Counter_Value"]) for r in rows if "k_gemv_plan" in r["Kernel_Name"]]
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
           "traffic_bytes": int((f_kib + w_kib) * 1024),
           "algorithmic_bytes": LAYERS * (q8_bytes(2 * HIDDEN, DIM) + q8_bytes(DIM, HIDDEN)),
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
    if len(sys.argv) > 2 and sys.argv[1] == "--write-checkpoint":
        # the configs[4] checkpoint, written ahead of a profiled --forward-only run
        smoe = importlib.import_module("smolmoe-c99_amd.smoe")
        smodel = importlib.import_module("smolmoe-c99_amd.model")
        smodel.synth_checkpoint(sys.argv[2], smoe.config_text(smoe.QWEN05), seed=4000, sigma=0.02, tied=True,
                                threads=min(16, len(os.sched_getaffinity(0))))
        log(f"bench: wrote {sys.argv[2]}")
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--q5-only":
        # configs[2] alone (the grouped Q5 GEMVs and batch-64 GEMMs): the program the Q5 rocprofv3 summary profiles
        log("bench: init", smq.init(0), smq.kernels_select())
        extra = {}

        def single(name, fn, nbytes, per_graph, reps=2, note=None):
            single_timing(extra, name, fn, nbytes, per_graph, reps, note)
        q5_extra(single, extra)
        print(json.dumps(extra), flush=True)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--anchor":
        # the HBM bandwidth and hand-off anchors alone (the program their rocprofv3 summary profiles)
        log("bench: init", smq.init(0), smq.kernels_select())
        extra = {}
        hbm_anchor(extra)
        handoff_anchor(extra)
        print(json.dumps(extra), flush=True)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--prefill-only":
        # the batched prefill GEMMs alone (configs[1] at batch 128, configs[3] at batch 64; exact and int8-MFMA):
        # the program the prefill rocprofv3 summaries profile
        log("bench: init", smq.init(0), smq.kernels_select())
        extra = {}
        prefill_only(extra)
        print(json.dumps(extra), flush=True)
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--forward-only":
        # configs[4] alone (no CPU leg): the program the decode-step rocprofv3 summaries profile;
        # --checkpoint PATH takes a file written by --write-checkpoint (and leaves it in place);
        # --decode-steps N times N greedy steps instead of 128; --runs R timed prefill + decode runs
        fp = argparse.ArgumentParser()
        fp.add_argument("--forward-only", action="store_true")
        fp.add_argument("--checkpoint", default=None)
        fp.add_argument("--decode-steps", type=int, default=128)
        fp.add_argument("--runs", type=int, default=FORWARD_RUNS)
        fa = fp.parse_args()
        log("bench: init", smq.init(0), smq.kernels_select())
        extra = {}
        model_forward_extra(argparse.Namespace(no_cpu=True, checkpoint=fa.checkpoint, decode_steps=fa.decode_steps,
                                               runs=fa.runs), extra)
        print(json.dumps(extra), flush=True)
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
    for _ in range(3):  # four LM-head copies in turn: 613 MB, past twice the 256 MB Infinity Cache
        head.append(smq.DeviceBuffer(head[0].nbytes))
        head[-1].copy_from(head[0])

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

    def gateup_group(m):
        """the 48 gate/up GEMVs of all layers (each layer's own activation): one launch"""
        smq.gemv_grouped([(layer.qmat(k), None, gu_out[l].ptr + (HIDDEN * 4 if k == "up" else 0), False,
                           ax[l].d, ax[l].q) for l, layer in enumerate(m) for k in ("gate", "up")])

    def down_group(m):
        smq.gemv_grouped([(layer.qmat("down"), None, y_out[l], False, ah[l].d, ah[l].q) for l, layer in enumerate(m)])

    def ffn_grouped(m):
        gateup_group(m)
        down_group(m)

    # the step's 72 GEMVs as one planned launch per model copy (the split over workgroups made once)
    plans = [smq.GemvPlan(ffn_items(m, ax, ah, gu_out, y_out)) for m in copies]

    def ffn_streamed(c):
        plans[c].launch()

    # one checked eager pass of each form (bounds checks on), then timing without host checks
    ffn_step(copies[0])
    smq.numeric_check()
    seq_layer0 = [gu_out[0].download(np.float32), y_out[0].download(np.float32)]
    for b in gu_out + y_out:
        b.fill(0)
    ffn_streamed(0)
    smq.numeric_check()
    smq.set_checks(False)
    step_bytes = LAYERS * (q8_bytes(2 * HIDDEN, DIM) + q8_bytes(DIM, HIDDEN))

    # headline: the 72 GEMVs of the 24-layer FFN step streamed in one planned launch; the K timed steps
    # (model copies alternating) are one captured graph, so no per-step graph launch gap sits between them
    if args.warmup:
        warm = smq.capture(lambda: [ffn_streamed(i % 2) for i in range(args.warmup)] and None)
        warm.launch()
    timed = smq.capture(lambda: [ffn_streamed(i % 2) for i in range(args.steps)] and None)
    # ms_per_step: the median of HEAD_SAMPLES replays of the K-step graph (best and all beside it)
    med, best, samples = timed_samples([timed], 1, HEAD_SAMPLES)
    ms_per_step = med / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    step_graphs = [smq.capture(lambda c=c: ffn_streamed(c)) for c in range(2)]
    per_graph_ms = timed_graph(step_graphs, args.steps)
    smq.numeric_check()
    gpu_layer0 = [gu_out[0].download(np.float32), y_out[0].download(np.float32)]  # for the CPU parity gate
    same_as_sequential = all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(gpu_layer0, seq_layer0))
    log(f"bench: FFN step streamed {ms_per_step * 1e3:.1f} us, {value:.0f} GB/s")
    # the same step as two grouped launches (48 gate/up, 24 down): the form before the plan
    two_graphs = [smq.capture(lambda: [ffn_grouped(copies[i % 2]) for i in range(args.steps)] and None)]
    timed_graph(two_graphs, 1)
    two_med, two_best, _ = timed_samples(two_graphs, 1, HEAD_SAMPLES)
    two_ms = two_med / args.steps
    log(f"bench: FFN step as two grouped launches {two_ms * 1e3:.1f} us")

    # the gate/up group alone (k_gemv_ct: coalesced 8-row x 28-block tiles, 236 MB), eight launches per graph
    # (the two copies alternating) so that one graph launch's host overhead is spread over eight
    per_graph = 8
    gu_graphs = [smq.capture(lambda: [gateup_group(copies[i % 2]) for i in range(per_graph)] and None)]
    timed_graph(gu_graphs, 2)
    reps = max(2, args.steps // 10)
    gu_med, gu_best, _ = timed_samples(gu_graphs, reps, HEAD_SAMPLES)
    gu_ms = gu_med / per_graph
    gu_bytes = LAYERS * q8_bytes(2 * HIDDEN, DIM)
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    log(f"bench: gate/up group {gu_ms * 1e3:.2f} us/launch, {gu_gbs:.0f} GB/s")

    # the same step as 48 dependent-order launches (as a decode must run them)
    seq_graphs = [smq.capture(lambda m=m: ffn_step(m)) for m in copies]
    timed_graph(seq_graphs, 4)
    seq_ms = timed_graph(seq_graphs, max(20, args.steps))
    one_ms = timed_graph([smq.capture(lambda m=m: gateup_only(m)) for m in copies], max(20, args.steps)) / LAYERS
    extra = {"headline_timing": {
        "what": "value = the 24-layer FFN step's 72 GEMVs as one planned launch (smq_gemv_plan: cross-layer "
                "grouped GEMV bandwidth, each GEMV with its own precomputed activation, so no layer waits for "
                "another); ms_per_step = median of the samples below, each one replay of the K-step graph",
        "samples_us_per_step": [round(t / args.steps * 1e3, 3) for t in samples],
        "median_us_per_step": round(med / args.steps * 1e3, 3), "best_us_per_step": round(best / args.steps * 1e3, 3),
        "best_GBps": round(step_bytes / (best / args.steps * 1e-3) / 1e9, 1)},
        "ffn_step_sequential": {
        "what": "the same 24-layer FFN step as 48 launches in layer order (gate+up fused, down), one graph",
        "us_per_step": round(seq_ms * 1e3, 2), "GBps": round(step_bytes / (seq_ms * 1e-3) / 1e9, 1),
        "gateup_single_launch_us": round(one_ms * 1e3, 3),
        "gateup_single_launch_GBps": round(q8_bytes(2 * HIDDEN, DIM) / (one_ms * 1e-3) / 1e9, 1),
        "bit_identical_to_streamed": same_as_sequential},
        "ffn_step_two_grouped_launches": {
            "what": "the same step as two grouped launches per step (smq_gemv_grouped: 48 gate/up, then 24 down)",
            "us_per_step": round(two_ms * 1e3, 2), "GBps": round(step_bytes / (two_ms * 1e-3) / 1e9, 1),
            "best_us_per_step": round(two_best / args.steps * 1e3, 2)},
        "gateup_group48": {
            "what": "the 48 gate/up GEMVs alone as one grouped launch (k_gemv_ct), eight launches per graph, "
                    "median of 11 replays",
            "us_per_launch": round(gu_ms * 1e3, 3), "GBps": round(gu_gbs, 1), "bytes_per_launch": gu_bytes,
            "pct_hbm_peak": round(100 * gu_gbs / HBM_PEAK_GBS, 1)},
        "ffn_step_streamed_graph_per_step": {
            "what": "the headline step, one graph launch per step (includes the gap between graph launches)",
            "us_per_step": round(per_graph_ms * 1e3, 2), "GBps": round(step_bytes / (per_graph_ms * 1e-3) / 1e9, 1)}}
    log(f"bench: FFN step sequential {seq_ms * 1e3:.1f} us")
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

        def single(name, fn, nbytes, per_graph, reps=2, note=None):
            single_timing(extra, name, fn, nbytes, per_graph, reps, note)

        single("c3_lm_head_gemv_151936x896",
               lambda i: smq.gemm_q8(head[i % 4], 28 * 36, ax[0].d, ax[0].q, VOCAB, 1, 28, logits, VOCAB),
               q8_bytes(VOCAB, DIM), 16, note="4 copies of 153 MB in turn (613 MB > 2 x 256 MB Infinity Cache)")
        single("c1_down_gemv_896x4864",
               lambda i: smq.matmul([(copies[i // LAYERS % 2][i % LAYERS].qmat("down"), None, y_out[0])], ah[0].d,
                                    ah[0].q, 1),
               q8_bytes(DIM, HIDDEN), 2 * LAYERS, note="48 distinct 4.9 MB matrices in turn (235 MB)")
        # prefill: exact GEMM and MFMA GEMM (f16 MFMA, activation in registers) at batch 128 on the fused gate+up shape
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
        # the single 896x896 Q8 GEMV (one launch; the 48 o-projections of the two copies in turn)
        single("c0_gemv_896x896",
               lambda i: smq.matmul([(copies[i // LAYERS % 2][i % LAYERS].qmat("o"), None, o_out)], ax[0].d,
                                    ax[0].q, 1),
               q8_bytes(DIM, Q_DIM), 2 * LAYERS, note="48 distinct 0.9 MB matrices in turn")
        # configs[0] streamed: one grouped launch of 48 distinct 896x896 GEMVs (each with one of the 24
        # layer activations), 576 matrices in turn (520 MB > twice the 256 MB Infinity Cache), as the
        # reference's tests/bench_matmul.c:112-117 rotates a matrix past the caches
        n0, g0 = 576, 48
        c0_bufs = [smq.DeviceBuffer(copies[0][0].dev["o"][0].nbytes) for _ in range(n0)]
        for k, b in enumerate(c0_bufs):
            b.copy_from(copies[k % 2][k // 2 % LAYERS].dev["o"][0])
        c0_out = [smq.DeviceBuffer(DIM * 4) for _ in range(g0)]

        def c0_grouped(i):
            base = (i % (n0 // g0)) * g0
            smq.gemv_grouped([(smq.QMat(c0_bufs[base + j], DIM, Q_DIM), None, c0_out[j], False, ax[j % LAYERS].d,
                               ax[j % LAYERS].q) for j in range(g0)])
        single("c0_gemv_896x896_grouped48", c0_grouped, g0 * q8_bytes(DIM, Q_DIM), n0 // g0,
               note="one launch of 48 distinct 896x896 GEMVs, 576 matrices (520 MB) in turn")
        smq.synchronize()
        one = smq.DeviceBuffer(DIM * 4)
        smq.matmul([(smq.QMat(c0_bufs[(n0 // g0 - 1) * g0 + 5], DIM, Q_DIM), None, one)], ax[5].d, ax[5].q, 1)
        extra["c0_gemv_896x896_grouped48"]["bit_identical_to_single"] = bool(np.array_equal(
            c0_out[5].download(np.float32).view(np.uint32), one.download(np.float32).view(np.uint32)))
        # the same matrices as planned launches of 192 GEMVs (smq_gemv_plan: more items than a grouped
        # launch takes, so a launch's fixed cost is spread over 173 MB); three plans in turn
        p0 = 192
        c0_pout = [smq.DeviceBuffer(DIM * 4) for _ in range(p0)]
        c0_plans = [smq.GemvPlan([(smq.QMat(c0_bufs[k * p0 + j], DIM, Q_DIM), None, c0_pout[j], False,
                                   ax[j % LAYERS].d, ax[j % LAYERS].q) for j in range(p0)]) for k in range(n0 // p0)]
        single("c0_gemv_896x896_plan192", lambda i: c0_plans[i % len(c0_plans)].launch(), p0 * q8_bytes(DIM, Q_DIM),
               n0 // p0 * 2, note="one planned launch of 192 distinct 896x896 GEMVs, 576 matrices (520 MB) in turn")
        smq.synchronize()
        smq.matmul([(smq.QMat(c0_bufs[(n0 // p0 - 1) * p0 + 7], DIM, Q_DIM), None, one)], ax[7].d, ax[7].q, 1)
        extra["c0_gemv_896x896_plan192"]["bit_identical_to_single"] = bool(np.array_equal(
            c0_pout[7].download(np.float32).view(np.uint32), one.download(np.float32).view(np.uint32)))
        for pl in c0_plans:
            pl.destroy()
        del c0_bufs
        # configs[1] down projection at batch 128 (exact GEMM; int8 MFMA)
        hx128 = Act(4200, 128, HIDDEN)
        dout = smq.DeviceBuffer(128 * DIM * 4)

        def prefill_down(i):
            layer = copies[i // LAYERS % 2][i % LAYERS]
            smq.matmul([(layer.qmat("down"), None, dout)], hx128.d, hx128.q, 128)

        single("c1_prefill_exact_gemm_896x4864_b128", prefill_down, q8_bytes(DIM, HIDDEN, 128), 8)
        smq.set_prefill_mfma(True)
        single("c1_prefill_mfma_gemm_896x4864_b128", prefill_down, q8_bytes(DIM, HIDDEN, 128), 24)
        smq.set_prefill_mfma(False)
        ops = 2 * DIM * HIDDEN * 128
        for k in ("c1_prefill_exact_gemm_896x4864_b128", "c1_prefill_mfma_gemm_896x4864_b128"):
            e = extra[k]
            e["int_TOPS"] = round(ops / (e["us"] * 1e-6) / 1e12, 2)
            e["pct_int8_peak"] = round(100 * ops / (e["us"] * 1e-6) / 5.0e15, 2)
        # configs[3] at batch 64 (exact GEMM; int8 MFMA)
        hx = Act(4100, 64, DIM)
        hout = smq.DeviceBuffer(64 * VOCAB * 4)
        single("c3_lm_head_gemm_151936x896_b64",
               lambda i: smq.gemm_q8(head[i % 4], 28 * 36, hx.d, hx.q, VOCAB, 64, 28, hout, VOCAB),
               q8_bytes(VOCAB, DIM, 64), 4)
        single("c3_lm_head_mfma_151936x896_b64",
               lambda i: smq.gemm_q8_mfma(head[i % 4], 28 * 36, hx.d, hx.q, VOCAB, 64, 28, hout, VOCAB),
               q8_bytes(VOCAB, DIM, 64), 8)
        del hout
        # the reference's own matmul benchmark shape (tests/bench_matmul.c:111-117): one Q8 matrix of 65536 rows x
        # 4864 (152 blocks, 342 MiB) against 1 token (decode GEMV) and 32 tokens (prefill); two copies alternate
        rb_rows, rb_nb = 65536, 152
        rb_host = np.tile(synth.q8_weights(7000, rb_rows // 64, rb_nb * 32), (64, 1))
        rb = [smq.DeviceBuffer.from_array(rb_host)]
        rb.append(smq.DeviceBuffer(rb[0].nbytes))
        rb[1].copy_from(rb[0])
        del rb_host
        rx = Act(7100, 32, rb_nb * 32)
        rout = smq.DeviceBuffer(32 * rb_rows * 4)
        single("refbench_gemv_65536x4864",
               lambda i: smq.gemm_q8(rb[i % 2], rb_nb * 36, rx.d, rx.q, rb_rows, 1, rb_nb, rout, rb_rows),
               q8_bytes(rb_rows, rb_nb * 32), 4,
               note="tests/bench_matmul.c's matrix (weights: 1/64 of the rows packed by the q8pack rule, repeated)")
        single("refbench_gemm_65536x4864_b32",
               lambda i: smq.gemm_q8(rb[i % 2], rb_nb * 36, rx.d, rx.q, rb_rows, 32, rb_nb, rout, rb_rows),
               q8_bytes(rb_rows, rb_nb * 32, 32), 4)
        single("refbench_mfma_65536x4864_b32",
               lambda i: smq.gemm_q8_mfma(rb[i % 2], rb_nb * 36, rx.d, rx.q, rb_rows, 32, rb_nb, rout, rb_rows),
               q8_bytes(rb_rows, rb_nb * 32, 32), 4)
        for k in ("refbench_gemv_65536x4864", "refbench_gemm_65536x4864_b32", "refbench_mfma_65536x4864_b32"):
            e = extra[k]
            ntok = 1 if "gemv" in k else 32
            e["weight_GBps"] = round(rb_rows * rb_nb * 36 / (e["us"] * 1e-6) / 1e9, 1)
            e["tok_s_eq_556MiB"] = round(ntok / (556 * 2 ** 20 / (rb_rows * rb_nb * 36) * e["us"] * 1e-6), 1)
        del rb, rout
        q5_extra(single, extra)
        hbm_anchor(extra)
        handoff_anchor(extra)

    if not args.no_extra:
        model_forward_extra(args, extra)

    cpu = None
    if not args.no_cpu:
        try:
            acts_x = [(synth_q(ax[l], DIM)) for l in range(LAYERS)]
            acts_h = [(synth_q(ah[l], HIDDEN)) for l in range(LAYERS)]
            ncpu = len(os.sched_getaffinity(0))
            threads = min(16, ncpu)
            kind, name, res, gate = cpu_baseline(copies[0], acts_x, acts_h, sorted({1, threads}), args.cpu_budget,
                                                 gpu_layer0)
            best, nreps, med_s = res[threads]
            phys, logical = physical_cores()
            cpu = {"value": round(step_bytes / best / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": kind,
                   "threads": threads, "physical_cores_visible": phys, "logical_cpus_visible": logical,
                   "median_value": round(step_bytes / med_s / 1e9, 2),
                   "gpu_bit_identical_layer0": gate,
                   "sample": f"{name}: {nreps} passes over the same 24-layer FFN decode step (353 MB of Q8 weights, "
                             f"best pass {best * 1e3:.2f} ms, median {med_s * 1e3:.2f} ms); 1 thread: "
                             f"{step_bytes / res[1][0] / 1e9:.2f} GB/s; "
                             f"host {cpu_model()}, {ncpu} CPUs visible, rows split statically, caller is worker 0"}
            log(f"bench: cpu {cpu['value']} GB/s on {threads} threads ({kind})")
        except Exception as ex:  # the CPU leg must not hide the GPU result
            log(f"bench: cpu baseline failed: {ex!r}")

    traffic = None
    tfile = os.path.join(ROOT, "profiles", "gemv_plan_q8_ffn_step_traffic.json")
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
                               "(gate 4864x896, up 4864x896, down 896x4864 per layer, each with its layer's "
                               "activation), 354 MB/step streamed as one planned launch of the 72 GEMVs, "
                               "2 model copies alternated", "bytes_per_step": step_bytes,
                   "parallelism": "none (1 GPU)"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "decode_tok_s": extra.get("c4_qwen05_forward", {}).get("decode_tok_s"),
        "roofline": {"kernel": "k_gemv_plan<exact>: the FFN step's 72 GEMVs in one launch, 768 workgroups (3 per "
                               "CU) split by bytes; 4864x896 items on coalesced 8-row x 28-block tiles (two in "
                               "flight), 896x4864 items on 14-row x 32-block K chunks; HIP events over the K-step "
                               "graph on the launch stream, median of 11 replays",
                     "bound": "hbm",
                     "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": step_bytes, "us_per_launch": round(ms_per_step * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
        "wall_s": round(time.time() - t_start, 1),
    }
    print(json.dumps(line), flush=True)


def model_forward_extra(args, extra):
    """the whole Qwen2.5-0.5B-shaped decoder (random-init Q8 weights,
    tied head) through the device-resident forward: prefill 512 random ids in
    one batch, then 128 greedy decode steps replayed as captured graphs. With
    the reference's own model layer built (oracle/_ref), the same checkpoint on
    the host cores gives the CPU rate and the parity gate (logits after the
    prompt, the first greedy tokens)."""
    import tempfile
    smoe = importlib.import_module("smolmoe-c99_amd.smoe")
    smodel = importlib.import_module("smolmoe-c99_amd.model")
    ncpu = len(os.sched_getaffinity(0))
    given = getattr(args, "checkpoint", None)
    nsteps = getattr(args, "decode_steps", 128)
    path = given or os.path.join(tempfile.gettempdir(), f"smq_bench_qwen05_{os.getpid()}.smoe")
    try:
        t0 = time.time()
        if not given:
            smodel.synth_checkpoint(path, smoe.config_text(smoe.QWEN05), seed=4000, sigma=0.02, tied=True,
                                    threads=min(16, ncpu))
        t_synth = time.time() - t0
        smq.set_checks(True)
        m = smodel.Model(path, context=1024, batch=512, logit_rows=1)
        banned = np.zeros(smoe.QWEN05["vocab_size"], np.uint8)
        banned[256] = 1  # BOS (sampler.c:57-63 skips banned ids)
        m.set_banned(banned)
        prompt = np.random.default_rng(3000).integers(0, smoe.QWEN05["vocab_size"], 512).astype(np.uint32)
        m.forward(prompt, 0, smodel.LOGITS_LAST)  # warm-up: first launches, graph capture
        m.generate(512, 5)
        smq.set_checks(False)
        # each run: the prefill (which drops the captured decode step), the decode step captured again
        # (untimed), then the greedy steps as graph replays
        nruns = getattr(args, "runs", FORWARD_RUNS)
        runs = []
        for _ in range(nruns):
            t0 = time.time()
            m.forward(prompt, 0, smodel.LOGITS_LAST)
            t1 = time.time()
            gl = m.logits(1)
            m.prepare_decode()
            t1b = time.time()
            toks = m.generate(512, nsteps + 1)
            t2 = time.time()
            runs.append((t1 - t0, t2 - t1b))
        pre_s = float(np.median([r[0] for r in runs]))
        dec_s = float(np.median([r[1] for r in runs]))
        pre_best, dec_best = min(r[0] for r in runs), min(r[1] for r in runs)
        smq.set_prefill_mfma(True)
        t0 = time.time()
        m.forward(prompt, 0, smodel.LOGITS_LAST)
        mfma_s = time.time() - t0
        smq.set_prefill_mfma(False)
        e = {"what": "Qwen2.5-0.5B shape (24 layers, 896/4864, GQA 14/2, vocab 151936, tied), random-init Q8, "
                     f"prefill 512 ids in one batch then {nsteps} greedy decode steps (HIP graph per step), BOS banned",
             "decode_tok_s": round(nsteps / dec_s, 1), "decode_ms_per_token": round(dec_s / nsteps * 1e3, 3),
             "prefill_tok_s": round(512 / pre_s, 1), "prefill_ms": round(pre_s * 1e3, 2),
             "timing": f"median of {nruns} runs (prefill, then the decode steps); best: decode "
                       f"{nsteps / dec_best:.1f} tok/s, prefill {512 / pre_best:.1f} tok/s",
             "prefill_mfma_tok_s": round(512 / mfma_s, 1),
             "prefill_mfma_note": "MFMA prefill (f16 MFMA on the 896-wide Q8 rows, int8 MFMA on the others): exact block sums applied in block order (the relaxed contract, within 1e-5; not bit-exact to the eight-lane one)",
             "decode_roofline_tok_s": round(8e12 / 555.7e6, 1), "weights_bytes_per_token": 555706368,
             "synth_s": round(t_synth, 2), "first_tokens": toks[:8].tolist()}
        del m
        if not args.no_cpu:
            import oracle
            if oracle.ReferenceModel.available():
                th = min(16, ncpu)
                try:  # the AVX2 kernels BASELINE names (kernels_select would pick VNNI where the host has it)
                    r = oracle.ReferenceModel(path, context=1024, batch=512, logit_rows=1, threads=th, avx2=True)
                except RuntimeError:
                    r = oracle.ReferenceModel(path, context=1024, batch=512, logit_rows=1, threads=th)
                r.set_banned(banned)
                cpu_runs = []
                for _ in range(CPU_FORWARD_RUNS):  # prefill 512, then 8 decode steps, each run timed
                    t0 = time.time()
                    r.prefill(prompt, 0, True)
                    t1 = time.time()
                    rl = r.logits(1)
                    rt = r.generate(512, 9)
                    t2 = time.time()
                    cpu_runs.append((t1 - t0, t2 - t1))
                cpre = [x[0] for x in cpu_runs]
                cdec = [x[1] for x in cpu_runs]
                phys, logical = physical_cores()
                e["cpu_reference"] = {"kind": "reference", "backend": r.backend, "threads": th,
                                      "physical_cores_visible": phys, "logical_cpus_visible": logical,
                                      "cpu": cpu_model(),
                                      "prefill_tok_s": round(512 / float(np.median(cpre)), 1),
                                      "decode_tok_s": round(8 / float(np.median(cdec)), 2),
                                      "prefill_tok_s_best": round(512 / min(cpre), 1),
                                      "decode_tok_s_best": round(8 / min(cdec), 2),
                                      "sample": "the reference's own model_forward (src/model.c built from its "
                                                f"sources) on the same checkpoint: {CPU_FORWARD_RUNS} runs of "
                                                "prefill 512 + 8 decode steps; medians, best beside them"}
                e["gpu_logits_bit_identical"] = bool(np.array_equal(gl.view(np.uint32), rl.view(np.uint32)))
                e["gpu_tokens_identical_first9"] = toks[:9].tolist() == rt.tolist()
                r.close()
        extra["c4_qwen05_forward"] = e
        log(f"bench: qwen0.5B forward: prefill {e['prefill_tok_s']} tok/s, decode {e['decode_tok_s']} tok/s")
    except Exception as ex:  # the model leg must not hide the matmul result
        log(f"bench: model forward leg failed: {ex!r}")
    finally:
        if not given and os.path.exists(path):
            os.remove(path)


def q5_extra(single, extra):
    """Qwen2.5-1.5B-shaped Q5 matmuls 8960x1536 and 1536x8960, each as one grouped launch of 16
    matrices with their own activations (two sets of 16 distinct 9.5 MB buffers alternated: 606 MB, past the
    Infinity Cache; the weights are an eighth of the rows packed by the Q5 rule and repeated, which changes no
    byte count), one matrix at batch 64 (exact GEMM, int8 MFMA); checks a grouped output against its
    single-matrix launch bit for bit."""
    n5 = 16
    shapes = {"gate": (8960, 1536), "down": (1536, 8960)}
    mats, acts, outs = {}, {}, {}
    for k, (name, (rows, cols)) in enumerate(shapes.items()):
        w = np.tile(synth.q5_weights(6000 + k, rows // 8, cols), (8, 1))  # an eighth of the rows, repeated
        bufs = [smq.DeviceBuffer.from_array(w) for _ in range(2 * n5)]
        mats[name] = [smq.QMat(b, rows, cols, smq.DTYPE_Q5) for b in bufs]
        acts[name] = [Act(6100 + 32 * k + i, 1, cols) for i in range(n5)]
        outs[name] = [smq.DeviceBuffer(rows * 4) for _ in range(n5)]
    for name, (rows, cols) in shapes.items():
        def grouped(i, name=name):
            base = (i % 2) * n5
            smq.gemv_grouped([(mats[name][base + j], None, outs[name][j], False, acts[name][j].d, acts[name][j].q)
                              for j in range(n5)])
        nbytes = n5 * q8_bytes(rows, cols, block=22)
        single(f"c2_q5_gemv_{rows}x{cols}_group{n5}", grouped, nbytes, 8,
               note=f"one launch of {n5} matrices with their own activations; two sets alternated (606 MB)")
        smq.synchronize()
        got = outs[name][3].download(np.float32)
        one = smq.DeviceBuffer(rows * 4)
        smq.matmul([(mats[name][3], None, one)], acts[name][3].d, acts[name][3].q, 1)
        extra[f"c2_q5_gemv_{rows}x{cols}_group{n5}"]["bit_identical_to_single"] = bool(
            np.array_equal(got.view(np.uint32), one.download(np.float32).view(np.uint32)))
    bx = Act(6500, 64, 1536)
    bout = smq.DeviceBuffer(64 * 8960 * 4)
    nb = 1536 // 32
    single("c2_q5_gemm_8960x1536_b64",
           lambda i: smq.gemm_q5(mats["gate"][i % (2 * n5)].buf, nb * 22, bx.d, bx.q, 8960, 64, nb, bout, 8960),
           q8_bytes(8960, 1536, 64, block=22), 8)
    single("c2_q5_mfma_8960x1536_b64",
           lambda i: smq.gemm_q5_mfma(mats["gate"][i % (2 * n5)].buf, nb * 22, bx.d, bx.q, 8960, 64, nb, bout, 8960),
           q8_bytes(8960, 1536, 64, block=22), 8)
    hx = Act(6600, 64, 8960)
    hout = smq.DeviceBuffer(64 * 1536 * 4)
    nbh = 8960 // 32
    single("c2_q5_gemm_1536x8960_b64",
           lambda i: smq.gemm_q5(mats["down"][i % (2 * n5)].buf, nbh * 22, hx.d, hx.q, 1536, 64, nbh, hout, 1536),
           q8_bytes(1536, 8960, 64, block=22), 8)
    single("c2_q5_mfma_1536x8960_b64",
           lambda i: smq.gemm_q5_mfma(mats["down"][i % (2 * n5)].buf, nbh * 22, hx.d, hx.q, 1536, 64, nbh, hout,
                                      1536),
           q8_bytes(1536, 8960, 64, block=22), 8)
    ops = 2 * 8960 * 1536 * 64
    for k in ("c2_q5_gemm_8960x1536_b64", "c2_q5_mfma_8960x1536_b64", "c2_q5_gemm_1536x8960_b64",
              "c2_q5_mfma_1536x8960_b64"):
        e = extra[k]
        e["int_TOPS"] = round(ops / (e["us"] * 1e-6) / 1e12, 2)
        e["pct_int8_peak"] = round(100 * ops / (e["us"] * 1e-6) / 5.0e15, 2)


def hbm_anchor(extra, gib=2):
    """What this device's HBM delivers to plain kernels (smq_stream_read / smq_stream_copy: coalesced
    16-byte pieces, grid-stride, eight in flight per thread) over a `gib` GiB buffer, swept over launch
    shapes; each shape is a graph of 4 launches timed 5 times (median of the samples), the best
    shape reported with the whole sweep beside it. Then the best read shape over the byte count of each
    grouped GEMV launch bench.py reports (one launch per region, the launch's fixed cost included)."""
    nbytes = gib << 30
    src = smq.DeviceBuffer(nbytes)
    src.fill(1)
    dst = smq.DeviceBuffer(nbytes // 2)
    sink = smq.DeviceBuffer(4)
    smq.synchronize()
    sweep = {}
    for nt in (True, False):
        for threads in (256, 512, 1024):
            for wgs in (256, 512, 1024, 2048, 4096):
                if wgs * threads > 4096 * 512:
                    continue
                g = [smq.capture(lambda: [smq.stream_read(src, nbytes, wgs, threads, nt, sink) for _ in range(4)]
                                 and None)]
                timed_graph(g, 1)
                med, best, _ = timed_samples(g, 1, 5)
                sweep[f"read_{'nt' if nt else 'plain'}_{wgs}x{threads}"] = round(nbytes * 4 / (med * 1e-3) / 1e9, 1)
    copy = {}
    half = nbytes // 2
    for nt in (True, False):
        for threads, wgs in ((256, 1024), (512, 1024), (512, 2048), (1024, 1024)):
            g = [smq.capture(lambda: [smq.stream_copy(dst, src, half, wgs, threads, nt) for _ in range(4)] and None)]
            timed_graph(g, 1)
            med, best, _ = timed_samples(g, 1, 5)
            copy[f"copy_{'nt' if nt else 'plain'}_{wgs}x{threads}"] = round(2 * half * 4 / (med * 1e-3) / 1e9, 1)
    best_read = max(sweep, key=sweep.get)
    best_copy = max(copy, key=copy.get)
    # the same read at the byte counts of single grouped launches: one launch per region, up to eight
    # distinct regions of the buffer per graph (no region is read twice in a row), so the launch's fixed
    # cost is in the rate
    rshape = best_read.split("_")
    rnt, (rwgs, rthr) = rshape[1] == "nt", map(int, rshape[2].split("x"))
    sized = {}
    for name, size in (("c0_group48_896x896", 48 * q8_bytes(DIM, DIM)),
                       ("c0_plan192_896x896", 192 * q8_bytes(DIM, DIM)),
                       ("down_group24_896x4864", LAYERS * q8_bytes(DIM, HIDDEN)),
                       ("q5_group16_8960x1536", 16 * q8_bytes(8960, 1536, block=22)),
                       ("gateup_group48_4864x896", 2 * LAYERS * q8_bytes(HIDDEN, DIM)),
                       ("ffn_step_plan72", LAYERS * (q8_bytes(2 * HIDDEN, DIM) + q8_bytes(DIM, HIDDEN)))):
        size = size // 256 * 256
        nreg = min(8, nbytes // size)  # distinct regions inside the buffer
        g = [smq.capture(lambda: [smq.stream_read(src.at(k * size), size, rwgs, rthr, rnt, sink)
                                  for k in range(nreg)] and None)]
        timed_graph(g, 1)
        med, best, _ = timed_samples(g, 1, 11)
        sized[name] = {"bytes": size, "us": round(med * 1e3 / nreg, 2),
                       "GBps": round(size * nreg / (med * 1e-3) / 1e9, 1), "regions": nreg}
    del src, dst
    extra["hbm_anchor"] = {
        "what": f"plain coalesced 16-byte streaming kernels over {gib} GiB (read: nothing written; copy: bytes read "
                "+ bytes written), medians of 5 samples of 4 graph-captured launches, per launch shape "
                "(workgroups x threads)",
        "read_GBps": sweep[best_read], "read_shape": best_read,
        "read_pct_hbm_peak": round(100 * sweep[best_read] / HBM_PEAK_GBS, 1),
        "copy_GBps": copy[best_copy], "copy_shape": best_copy,
        "read_at_launch_sizes": sized,
        "read_sweep": sweep, "copy_sweep": copy}
    log(f"bench: HBM anchor read {sweep[best_read]} GB/s ({best_read}), copy {copy[best_copy]} GB/s ({best_copy}); "
        f"one read launch of a grouped GEMV's bytes: " + ", ".join(f"{k} {v['us']} us {v['GBps']} GB/s"
                                                                for k, v in sized.items()))


def handoff_anchor(extra, episodes=200):
    """What a hand-off between dependent phases costs: a grid barrier among resident workgroups (one per
    CU; smq_grid_barrier_probe, kinds 0-2, at 64/128/256 workgroups: (launch with `episodes` barriers -
    launch with none) / episodes, best of 5 each), against the dependent-launch gap of a graph of 200
    small kernels (smq_stream_read of 16 KiB at 64/256/1024 workgroups: replay time / 200, best of 5)."""
    kinds = {0: "one_counter", 1: "per_xcd_counters", 2: "per_workgroup_flags"}
    cus = {}
    for kind, kname in kinds.items():
        for wgs in (64, 128, 256):
            t0 = min(smq.grid_barrier_probe(wgs, 0, kind) for _ in range(5))
            t1 = min(smq.grid_barrier_probe(wgs, episodes, kind) for _ in range(5))
            cus[f"{kname}_{wgs}wg_us"] = round((t1 - t0) * 1e3 / episodes, 3)
    buf = smq.DeviceBuffer(16384)
    sink = smq.DeviceBuffer(4)
    gaps = {}
    for wgs in (64, 256, 1024):
        g = [smq.capture(lambda: [smq.stream_read(buf, 16384, wgs, 64, False, sink) for _ in range(200)] and None)]
        timed_graph(g, 1)
        gaps[f"{wgs}wg_us"] = round(min(timed_graph(g, 1) for _ in range(5)) * 1e3 / 200, 3)
    del buf, sink
    extra["handoff_anchor"] = {
        "what": "cost of one hand-off between dependent phases: a grid barrier among resident workgroups (one per "
                "CU, agent-scope release/acquire, bounded waits) against a dependent kernel launch inside a "
                "HIP graph; best of 5",
        "grid_barrier": cus, "graph_launch_gap": gaps}
    log(f"bench: hand-off anchor: barrier {cus}, graph launch gap {gaps}")


def prefill_only(extra):
    """configs[1] gate/up 9728x896 and down 896x4864 at batch 128, configs[3] 151936x896 at batch 64: each as
    a graph of launches over two weight copies, exact GEMM and int8-MFMA GEMM."""
    def single(name, fn, nbytes, ops, per_graph, reps=2):
        single_timing(extra, name, fn, nbytes, per_graph, reps)
        us = extra[name]["us"]
        extra[name]["int_TOPS"] = round(ops / (us * 1e-6) / 1e12, 2)
        extra[name]["pct_int8_peak"] = round(100 * ops / (us * 1e-6) / 5.0e15, 2)

    shapes = {"gate_up": (2 * HIDDEN, DIM, 128), "down": (DIM, HIDDEN, 128), "lm_head": (VOCAB, DIM, 64)}
    for name, (rows, cols, ntok) in shapes.items():
        nb = cols // 32
        w = synth.q8_weights(8000 + rows, rows if rows < 20000 else rows // 16, cols)
        if rows >= 20000:
            w = np.tile(w, (16, 1))
        bufs = [smq.DeviceBuffer.from_array(w) for _ in range(2)]
        x = Act(8100 + cols, ntok, cols)
        out = smq.DeviceBuffer(ntok * rows * 4)
        nbytes, ops = q8_bytes(rows, cols, ntok), 2 * rows * cols * ntok
        single(f"{name}_exact_{rows}x{cols}_b{ntok}",
               lambda i: smq.gemm_q8(bufs[i % 2], nb * 36, x.d, x.q, rows, ntok, nb, out, rows), nbytes, ops, 4)
        single(f"{name}_mfma_{rows}x{cols}_b{ntok}",
               lambda i: smq.gemm_q8_mfma(bufs[i % 2], nb * 36, x.d, x.q, rows, ntok, nb, out, rows), nbytes, ops, 8)
        del bufs, out


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
