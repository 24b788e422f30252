#!/usr/bin/env python3
"""Benchmark of the fp32 training path on one MI355X.

Prints ONE JSON line. The headline workload is the largest configuration that fits one GPU,
the scaled Transformer training step (12 pre-LN blocks, d_model
1024, 16 heads, FFN 4096, context 512, byte vocabulary 256, batch 16, causal; forward,
backward and Adam lr 1e-3) on a resident synthetic batch, from seeded parameters drawn with
the reference's initialisers (workloads.py; the same ones tests/test_cfg5_parity.py checks
against the compiled reference). `value` is training steps per second through the C++ engine,
timed with HIP events on the engine's stream over exactly --steps steps after --warmup
untimed steps; every step also carries its own event pair, for the median.

The same line carries:
  roofline      the step's dominant kernel, the MFMA weight-gradient products dW = X^T dY
                (gemm_kernel<128,128,32,64,32,true,false>), timed live at their in-step
                shapes with HIP events, against the fp32 MFMA peak;
  cpu_baseline  the reference engine compiled from its own sources (oracle/_ref) running one
                whole training step of the same model on the host cores (about 40 s);
  extra         the other configurations: cfg 2 CNN and cfg 3 char-Transformer steps (each
                with its own reference CPU baseline), cfg 1 GEMMs (512^3 and 4096^3), cfg 4
                bandwidth kernels and the path's other bandwidth kernels, each with its
                roofline fraction.

The line is compacted (compact()) to about 4 KB so that a log tail keeps all of it;
--full-out FILE writes the uncompacted record (per-mode GEMM timings, per-shape details).

Only the cpu_baseline legs touch oracle/ (through tests/_oracle.py), as the reference being
timed; nothing measured on the GPU goes through it.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "cpp-ai-engine_amd")
sys.path.insert(0, PKG)

import workloads as W  # noqa: E402

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def metric_name():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


# Seeds of the synthetic workloads (workloads.py); the cfg 5 ones are the parity test's.
CFG5_PARAM_SEED, LM_INPUT_SEED = 11, 3


# ------------------------------------------------------------------ timing

class Timer:
    """HIP events on the stream the engine launches on (torch's default stream is the
    null stream, which is also the engine's)."""

    def __init__(self, torch):
        self.torch = torch
        assert torch.cuda.current_stream().cuda_stream == 0, "expected the null stream"

    def time(self, fn, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e-3 / steps  # seconds per call

    def time_steps(self, fn, steps, warmup):
        """Exactly `steps` calls after `warmup` untimed ones, an event recorded before each
        call and after the last: (seconds for all of them, [seconds per call])."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for i in range(steps):
            fn()
            ev[i + 1].record()
        torch.cuda.synchronize()
        per = [ev[i].elapsed_time(ev[i + 1]) * 1e-3 for i in range(steps)]
        return ev[0].elapsed_time(ev[-1]) * 1e-3, per

    def time_batch(self, enqueue, reps, warmup):
        """enqueue(n) puts n launches on the stream from native code in one call, so the
        events see back-to-back kernels rather than Python's launch gaps."""
        torch = self.torch
        enqueue(warmup)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        enqueue(reps)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e-3 / reps

    def median_batch(self, enqueue, reps, warmup, repeats=15):
        """Median over `repeats` timed batches of time_batch (seconds per launch)."""
        t = [self.time_batch(enqueue, reps, warmup if i == 0 else 0) for i in range(repeats)]
        return float(np.median(t))


def roofline(name, bound, work, seconds, traffic=None):
    if bound == "hbm":
        achieved = work / seconds / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    else:
        achieved = work / seconds / 1e12
        peak, unit = PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
    return {"kernel": name, "bound": bound, "achieved": round(achieved, 2), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
            "us_per_launch": round(seconds * 1e6, 3)}


def committed_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(kernel)


def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": usable}


def cpu_threads():
    """All host cores this process may use (BENCH_CPU_THREADS overrides)."""
    return int(os.environ.get("BENCH_CPU_THREADS", "0")) or host_info()["usable_cpus"] or 1


# ------------------------------------------------------------------ cfg 5 (headline)

def lm_step_flops(batch, seq, d, ff, vocab, layers):
    """Algorithmic FLOPs of one training step: every GEMM forward (2mnk) plus its two
    backward products; the full S x S scores are computed (the mask saves nothing)."""
    t = batch * seq
    per_block = 2 * t * d * d * 4 + 2 * t * d * ff * 2 + 2 * batch * seq * seq * d * 2
    fwd = layers * per_block + 2 * t * d * vocab
    return 3 * fwd


PROBE_STEPS = 3  # training steps after the timed ones with the dominant products probed


def cfg5_leg(engine_mod, eng, timer, steps, warmup, hip=None):
    """cfg 5 training steps through the engine: forward + backward + Adam on one resident
    batch; returns the record. With `hip`, PROBE_STEPS more steps run with the weight-gradient
    products bracketed by HIP events on their stream (ehip_gemm_probe_arm): the dominant
    kernel's time measured inside training steps, outside the timed ones so that their
    event records cannot touch `value`."""
    b, s, vocab, d, h, ff, layers = W.TRANSFORMER_CFG5
    params = W.lm_init_params(CFG5_PARAM_SEED, vocab, d, ff, layers)
    ids, targets = W.lm_inputs(LM_INPUT_SEED, b, s, vocab)
    tr = engine_mod.Trainer.charlm(eng, ids, targets, vocab, d, h, ff, layers, params, lr=1e-3)
    del params
    tr.step()
    first = tr.loss()
    total, per = timer.time_steps(tr.step, steps, max(warmup - 1, 0))
    last = tr.loss()
    n_params = int(tr.num_params())
    probe = None
    if hip is not None:
        shapes = [(m, n, k) for m, n, k, _ in cfg5_dw_shapes()]
        hip.gemm_probe_arm(True, False, shapes, 6 * layers * PROBE_STEPS + 16)
        for _ in range(PROBE_STEPS):
            tr.step()
        ms, products, flop = hip.gemm_probe_read()
        probe = {"ms": ms, "products": products, "flop": flop}
    tr.close()
    fl = lm_step_flops(b, s, d, ff, vocab, layers)
    sec = total / steps
    return {"seconds": sec, "median_s": float(np.median(per)), "params": n_params,
            "step_tflop": fl / 1e12, "loss_first_step": first, "loss_last": last,
            "per_step_ms": [round(x * 1e3, 3) for x in per], "dw_probe": probe}


def cfg5_dw_shapes():
    """The weight-gradient products of one cfg 5 block, dW = X^T dY with X (tokens, in) and
    dY (tokens, out): (in, out, tokens, count) for the query/key/value/output projections,
    ff1 and ff2. The engine's Linear backward issues exactly these ehip_gemm_f32 calls
    (trans_a = 1, beta = 0), 12 blocks per step."""
    b, s, _, d, _, ff, _ = W.TRANSFORMER_CFG5
    t = b * s
    return [(d, d, t, 4), (d, ff, t, 1), (ff, d, t, 1)]


def dominant_kernel(eng, timer, torch):
    """The cfg 5 step's largest kernel by total time (rocprofv3 --kernel-trace --stats of
    this benchmark, profiles/transformer_cfg5_kernels.md): the weight-gradient products,
    gemm_kernel<128,128,32,64,32,true,false> (A read transposed), 6 per block. Timed live at
    their in-step shapes as back-to-back launches from native code between HIP events on
    the engine's stream (median of 15 batches per shape); splitk_reduce launches, where the
    dispatcher splits K, are inside the timed region. Algorithmic FLOPs per block =
    sum over the six products of 2 * in * out * tokens = 206.2 GFLOP; `achieved` = that /
    the six products' summed time."""
    r = torch.Generator(device="cuda").manual_seed(6)
    flops, secs, shapes = 0.0, 0.0, {}
    for m, n, k, count in cfg5_dw_shapes():
        x = torch.randn(k, m, device="cuda", generator=r)
        dy = torch.randn(k, n, device="cuda", generator=r)
        dw = torch.empty(m, n, device="cuda")
        sec = timer.median_batch(lambda reps: eng.repeat_gemm(reps, x, dy, dw, trans_a=True),
                                 10, 3)
        fl = 2.0 * m * n * k
        shapes[f"{m}x{n}x{k}"] = {"count_per_block": count, "us": round(sec * 1e6, 2),
                                  "tflops": round(fl / sec / 1e12, 2)}
        flops += count * fl
        secs += count * sec
        del x, dy, dw
    roof = roofline("gemm_kernel<128,128,32,64,32,true,false> (+splitk_reduce): cfg5 weight "
                    "gradients dW = X^T dY, one block's six products (4 x 1024x1024x8192, "
                    "1024x4096x8192, 4096x1024x8192)", "mfma", flops / 6, secs / 6,
                    committed_traffic("cfg5_dw_gemm"))
    roof["flop_per_launch"] = flops / 6
    roof["shapes"] = shapes
    return roof


def in_step_roofline(probe, leg):
    """The dominant kernel's roofline from the products timed inside training steps (the
    probe: summed event time of every weight-gradient product of PROBE_STEPS steps, its
    split-K reduction included), with the back-to-back leg's figures kept under "leg" (and
    its per-shape rates) for comparison."""
    if not probe or probe["products"] == 0:
        return leg
    roof = roofline(leg["kernel"], "mfma", probe["flop"] / probe["products"],
                    probe["ms"] * 1e-3 / probe["products"], leg["traffic"])
    roof["flop_per_launch"] = probe["flop"] / probe["products"]
    roof["launches"] = probe["products"]
    roof["shapes"] = leg["shapes"]
    roof["leg"] = {"achieved": leg["achieved"], "frac": leg["frac"],
                   "us_per_launch": leg["us_per_launch"]}
    return roof


def cpu_cfg5_baseline(sample_batch):
    """The cfg 5 step on the reference engine (oracle/_ref) on all host cores: the full
    12-block model from the same initial parameters, one training step (forward, backward,
    Adam). With sample_batch = 16 (the default) that is one whole step, timed as it is (about
    40 s on 16 threads). A smaller sample_batch times the step over that many of the 16
    sequences and scales it: the work is linear in the batch except the Adam update over the
    151.7 M parameters, timed on its own and counted once,
    t(16) = (16 / sample_batch) * (t(sample) - t(adam)) + t(adam)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _oracle import Ref
    b, s, vocab, d, h, ff, layers = W.TRANSFORMER_CFG5
    threads = cpu_threads()
    ref = Ref()
    ref.set_threads(threads)
    params = W.lm_init_params(CFG5_PARAM_SEED, vocab, d, ff, layers)
    ids, targets = W.lm_inputs(LM_INPUT_SEED, b, s, vocab)
    ids, targets = ids[:sample_batch], targets[:sample_batch * s]
    t0 = time.perf_counter()
    losses, _ = ref.charlm_train(ids, targets, vocab, d, h, ff, layers, params, 1, 1e-3)
    t_sample = time.perf_counter() - t0
    assert np.all(np.isfinite(losses))
    info = host_info()
    cpu = {"cores": threads, "kind": "reference", "cpu_model": info["cpu_model"],
           "nproc": info["nproc"]}
    if sample_batch >= b:
        return {"value": round(1.0 / t_sample, 5), "unit": "steps/s", **cpu,
                "sample": f"one whole cfg5 step (batch 16 x 512, fwd+bwd+Adam) of the reference "
                          f"engine (oracle/_ref, its sources, g++ -O3) on {threads} threads from "
                          f"the GPU run's initial parameters: {t_sample:.1f} s",
                "seconds_per_step": round(t_sample, 2)}
    g = np.full(params.size, 1e-3, np.float32)
    t0 = time.perf_counter()
    ref.adam_steps(params, g, 1e-3)
    t_adam = time.perf_counter() - t0
    t_full = (b / sample_batch) * (t_sample - t_adam) + t_adam
    return {"value": round(1.0 / t_full, 5), "unit": "steps/s", **cpu,
            "sample": f"cfg5 step of the reference engine (oracle/_ref) on {threads} threads over "
                      f"{sample_batch} of 16 sequences ({t_sample:.1f} s, Adam {t_adam:.1f} s), "
                      f"scaled to 16: {t_full:.1f} s",
            "seconds_per_step": round(t_full, 2)}


def cpu_matmul_threads(threads_list):
    """cfg 1 on the reference CPU path: C = A B at 512^3 on 1 thread and on all threads."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _oracle import Ref
    r = np.random.default_rng(512)
    a = r.standard_normal((512, 512), np.float32)
    b = r.standard_normal((512, 512), np.float32)
    ref = Ref()
    out = {}
    for t in threads_list:
        ref.set_threads(t)
        ref.matmul(a, b)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 1.0 or reps < 3:
            ref.matmul(a, b)
            reps += 1
        sec = (time.perf_counter() - t0) / reps
        out[f"{t}_threads"] = {"ms": round(sec * 1e3, 3),
                               "gflops": round(2 * 512 ** 3 / sec / 1e9, 2)}
    return out


# ------------------------------------------------------------------ cfg 2, cfg 3

def graph_mode(make, timer, steps, warmup, eager_loss):
    """The same training run with the trainer in graph mode (the second step captured into
    one HIP graph, every later one a single replay): the same number of steps as the eager
    leg, so the last loss must be the eager leg's, bit for bit."""
    tr = make()
    tr.set_graph(True)
    tr.step()
    total, per = timer.time_steps(tr.step, steps, warmup)
    last = tr.loss()
    tr.close()
    sec = total / steps
    return {"steps_per_s": round(1.0 / sec, 2), "ms_per_step": round(sec * 1e3, 4),
            "median_ms_per_step": round(float(np.median(per)) * 1e3, 4),
            "loss_last": round(last, 5), "loss_last_equals_eager": bool(last == eager_loss)}


def cnn_leg(engine_mod, eng, timer, steps, warmup):
    x, labels, params = W.cnn_inputs()
    make = lambda: engine_mod.Trainer.cnn(eng, x, labels, params, lr=1e-3)  # noqa: E731
    tr = make()
    tr.step()
    first = tr.loss()
    total, per = timer.time_steps(tr.step, steps, max(warmup - 1, 0))
    last = tr.loss()
    assert np.isfinite(first) and np.isfinite(last), (first, last)
    tr.close()
    sec = total / steps
    return {"steps_per_s": round(1.0 / sec, 2), "ms_per_step": round(sec * 1e3, 4),
            "median_ms_per_step": round(float(np.median(per)) * 1e3, 4),
            "loss_first_step": round(first, 5), "loss_last": round(last, 5),
            "graph": graph_mode(make, timer, steps, max(warmup - 1, 0), last)}


def cnn_dominant_kernel(eng, hip, timer, torch):
    """The cfg 2 step's largest kernel by total time (profiles/cnn_step_kernels.md): the
    backward of the fused conv2 block (Conv2d 8 -> 16, 3x3, pad 1 -> ReLU -> MaxPool2d 2 on a
    64 x 8 x 14 x 14 input) -- conv3_pool_backward and conv_weight_reduce -- timed as that
    launch pair. HBM-bound by its data, latency-bound at this size: algorithmic bytes = x,
    the pooled gradient, the pooled values, the argmax and the weights read once, dx, dW and
    db written once."""
    r = torch.Generator(device="cuda").manual_seed(5)
    x = torch.rand(64, 8, 14, 14, device="cuda", generator=r)
    w = torch.rand(16, 8, 3, 3, device="cuda", generator=r) * 0.6 - 0.3
    b = torch.zeros(16, device="cuda")
    out, am = hip.conv2d_relu_maxpool(x, w, b, 1, 1, 2)
    g = torch.randn(out.shape, device="cuda", generator=r)
    dx, dw, db = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
    cw, pw = hip.conv_relu_pool_windows(x.shape, w.shape, 1, 1, 2)
    sec = timer.median_batch(
        lambda n: eng.repeat_conv_relu_pool_backward(n, x, w, g, out, am, dw, db, cw, pw, dx=dx),
        100, 50)
    work = 4 * (2 * x.numel() + 3 * out.numel() + 2 * w.numel() + b.numel())
    return roofline("conv3_pool_backward+conv_weight_reduce (conv2 block dx/dW/db, "
                    "64x8x14x14, 16 filters 3x3, pool 2)", "hbm", work, sec,
                    committed_traffic("conv2_block_backward"))


def cpu_cnn_baseline(seconds_target):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _oracle import Ref
    x, labels, params = W.cnn_inputs()
    threads = cpu_threads()
    ref = Ref()
    ref.set_threads(threads)
    t0 = time.perf_counter()
    ref.cnn_train(x, labels, params, 2, 1e-3)
    per = (time.perf_counter() - t0) / 2
    n = max(3, min(2000, int(seconds_target / max(per, 1e-6))))
    t0 = time.perf_counter()
    losses, _ = ref.cnn_train(x, labels, params, n, 1e-3)
    dt = time.perf_counter() - t0
    assert np.all(np.isfinite(losses))
    return {"value": round(n / dt, 3), "unit": "steps/s", "cores": threads, "kind": "reference",
            "sample": f"cfg2 CNN training step (batch 64, Adam), {n} consecutive steps of the "
                      f"reference engine compiled from its own sources (oracle/_ref, -O3, no "
                      f"-march) on {threads} host threads, {dt:.1f} s"}


def cpu_charlm_baseline(ids, targets, dims, params, seconds_target):
    """The char-Transformer (cfg3) step of the reference engine itself on the host cores,
    from the same initial parameters as the GPU run; a bounded sample of steps."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _oracle import Ref
    vocab, d, h, ff, layers = dims
    threads = cpu_threads()
    ref = Ref()
    ref.set_threads(threads)
    t0 = time.perf_counter()
    ref.charlm_train(ids, targets, vocab, d, h, ff, layers, params, 1, 1e-3)
    per = time.perf_counter() - t0
    n = max(2, min(500, int(seconds_target / max(per, 1e-6))))
    t0 = time.perf_counter()
    losses, _ = ref.charlm_train(ids, targets, vocab, d, h, ff, layers, params, n, 1e-3)
    dt = time.perf_counter() - t0
    assert np.all(np.isfinite(losses))
    return {"value": round(n / dt, 3), "unit": "steps/s", "cores": threads, "kind": "reference",
            "sample": f"cfg3 char-Transformer step (batch 32 x 64, Adam), {n} consecutive steps "
                      f"of the reference engine compiled from its own sources (oracle/_ref, -O3, "
                      f"no -march) on {threads} host threads from the GPU run's initial "
                      f"parameters, {dt:.1f} s"}


def charlm_leg(engine_mod, eng, timer, cpu_seconds):
    b, s, vocab, d, h, ff, layers = W.CHARLM_CFG3
    ids, targets = W.lm_inputs(LM_INPUT_SEED, b, s, vocab)
    params = W.lm_init_params(CFG5_PARAM_SEED, vocab, d, ff, layers)
    make = lambda: engine_mod.Trainer.charlm(eng, ids, targets, vocab, d, h, ff,  # noqa: E731
                                             layers, params, lr=1e-3)
    tr = make()
    tr.step()
    first = tr.loss()
    total, per = timer.time_steps(tr.step, 100, 9)
    fl = lm_step_flops(b, s, d, ff, vocab, layers)
    sec = total / 100
    rec = {"steps_per_s": round(1.0 / sec, 3), "ms_per_step": round(sec * 1e3, 3),
           "median_ms_per_step": round(float(np.median(per)) * 1e3, 4),
           "params": int(tr.num_params()), "step_tflop": round(fl / 1e12, 4),
           "achieved_tflops": round(fl / sec / 1e12, 2),
           "frac_of_mfma_peak": round(fl / sec / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
           "loss_first_step": round(first, 5), "loss_last": round(tr.loss(), 5)}
    eager_last = tr.loss()
    tr.close()
    g = graph_mode(make, timer, 100, 9, eager_last)
    g["achieved_tflops"] = round(fl * g["steps_per_s"] / 1e12, 2)
    g["frac_of_mfma_peak"] = round(fl * g["steps_per_s"] / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)
    rec["graph"] = g
    if cpu_seconds > 0:
        log("bench: reference CPU baseline, cfg3")
        cpu = cpu_charlm_baseline(ids, targets, (vocab, d, h, ff, layers), params, cpu_seconds)
        rec["cpu_baseline"] = cpu
        rec["gpu_over_cpu"] = round(rec["steps_per_s"] / cpu["value"], 1)
    return rec


def bandwidth_legs(hip, eng, timer, torch, r, rows, d, sum_rows, ff, srows, scols, im_shape,
                   reps):
    """LayerNorm forward / backward (rows x d), the bias-gradient column sum (sum_rows x ff),
    softmax forward / backward (srows x scols) and max-pool forward / backward (k 2 over
    im_shape), each as `reps` back-to-back native launches, median of 15 batches."""
    bl = {}
    med = lambda op, ts, ext=(), f=0.0, w=None: timer.median_batch(
        lambda q: eng.repeat_bandwidth(q, op, ts, ext, f, w), reps, 3)
    x = torch.randn(rows, d, device="cuda", generator=r)
    gam = torch.randn(d, device="cuda", generator=r)
    bet = torch.randn(d, device="cuda", generator=r)
    y, xh, inv = hip.layernorm(x, gam, bet)
    n = x.numel()
    sec = med("layernorm", [x, gam, bet, y, xh, inv], (rows, d), 1e-5)
    bl[f"layernorm {rows}x{d}"] = roofline("layernorm", "hbm", 12 * n + 4 * rows, sec)
    dx = torch.empty_like(x)
    dg, db = torch.empty(d, device="cuda"), torch.empty(d, device="cuda")
    sec = med("layernorm_backward", [x, xh, gam, inv, dx, dg, db], (rows, d))
    bl[f"layernorm_backward {rows}x{d}"] = roofline("layernorm_backward", "hbm",
                                                    12 * n + 4 * rows + 8 * d, sec)
    # As the engine runs it inside a step: the row kernel with the group partials; the
    # dgamma / dbeta sums of all LayerNorms (and convolution blocks) of a backward run later
    # in one launch of their own, or inside Adam's.
    import ctypes
    groups = ctypes.c_int64(0)
    nparts = hip.lib.ehip_layernorm_backward_partials(rows, d, ctypes.byref(groups))
    if nparts > 0:
        part = torch.empty(nparts, device="cuda")
        sec = med("layernorm_backward_rows", [x, xh, gam, inv, dx, part], (rows, d, groups.value))
        bl[f"layernorm_backward {rows}x{d} (engine: sums deferred)"] = roofline(
            "layernorm_backward_rows", "hbm", 12 * n + 4 * rows + 4 * d, sec)
        if d <= 1024:  # dx added into the residual stream's gradient (reads it too)
            sec = med("layernorm_backward_rows_acc", [x, xh, gam, inv, dx, part],
                      (rows, d, groups.value))
            bl[f"layernorm_backward {rows}x{d} (engine: accumulating dx)"] = roofline(
                "layernorm_backward_rows", "hbm", 16 * n + 4 * rows + 4 * d, sec)
        del part
    del x, y, xh, inv, dx
    torch.cuda.empty_cache()
    gb = torch.randn(sum_rows, ff, device="cuda", generator=r)
    colsum = torch.empty(ff, device="cuda")
    sec = med("sum_axis", [gb, colsum], (1, sum_rows, ff))
    bl[f"bias_grad_sum {sum_rows}x{ff}"] = roofline("sum_axis", "hbm", 4 * gb.numel() + 4 * ff, sec)
    del gb
    sc = torch.randn(srows, scols, device="cuda", generator=r)
    sy = torch.empty_like(sc)
    sec = med("softmax", [sc, sy], (srows, scols))
    bl[f"softmax {srows}x{scols}"] = roofline("softmax", "hbm", 8 * sc.numel(), sec)
    sdx = torch.empty_like(sc)
    sec = med("softmax_backward", [sy, sc, sdx], (srows, scols))
    bl[f"softmax_backward {srows}x{scols}"] = roofline("softmax_backward", "hbm",
                                                       12 * sc.numel(), sec)
    del sc, sy, sdx
    torch.cuda.empty_cache()
    im = torch.randn(*im_shape, device="cuda", generator=r)
    pooled, am = hip.maxpool(im, 2, 2)
    w = ehip_window(im_shape)
    sec = med("maxpool", [im, pooled, am], (), 0.0, w)
    shape = "x".join(str(v) for v in im_shape)
    bl[f"maxpool {shape} k2"] = roofline("maxpool", "hbm", 6 * im.numel(), sec)
    gp = torch.randn_like(pooled)
    dim = torch.empty_like(im)
    sec = med("maxpool_backward", [am, gp, dim], (), 0.0, w)
    bl[f"maxpool_backward {shape} k2"] = roofline("maxpool_backward", "hbm", 6 * im.numel(), sec)
    del im, pooled, am, gp, dim
    return bl


def ehip_window(im_shape, k=2, stride=2, pad=0):
    import ehip
    return ehip.window(*im_shape, k, k, stride, pad)


def extras(hip, eng, engine_mod, timer, torch, cpu_seconds=0.0):
    out = {}
    # cfg 2 and cfg 3: the launch-bound training steps, each with its reference CPU baseline.
    log("bench: cfg2 CNN training step")
    out["cnn_cfg2"] = cnn_leg(engine_mod, eng, timer, 200, 20)
    out["cnn_cfg2"]["roofline"] = cnn_dominant_kernel(eng, hip, timer, torch)
    if cpu_seconds > 0:
        log("bench: reference CPU baseline, cfg2")
        cpu = cpu_cnn_baseline(cpu_seconds)
        out["cnn_cfg2"]["cpu_baseline"] = cpu
        out["cnn_cfg2"]["gpu_over_cpu"] = round(out["cnn_cfg2"]["steps_per_s"] / cpu["value"], 1)
    log("bench: cfg3 char-Transformer training step")
    out["charlm_cfg3"] = charlm_leg(engine_mod, eng, timer, cpu_seconds)
    # cfg 1: C = A B and its backward (dA = dC B^T, dB = A^T dC) at 512^3 (805.3 MFLOP per
    # trio), and 4096^3. The backward is one ehip_matmul_backward_f32 call (both products in
    # one launch where they take the K-sliced tiles, as the engine's matmul backward runs
    # them); the two products launched one by one are recorded beside it.
    for n in (512, 4096):
        r = torch.Generator(device="cuda").manual_seed(n)
        a = torch.randn(n, n, device="cuda", generator=r)
        b = torch.randn(n, n, device="cuda", generator=r)
        dc = torch.randn(n, n, device="cuda", generator=r)
        c, da, db = (torch.empty(n, n, device="cuda") for _ in range(3))
        fl = 2.0 * n ** 3
        reps, warm = (20, 3) if n == 4096 else (200, 20)
        modes = {
            "fwd C=AB": (fl, lambda q: eng.repeat_gemm(q, a, b, c)),
            "bwd dA and dB (one call)": (2 * fl, lambda q: eng.repeat_matmul_backward(
                q, a, b, dc, da, db)),
            "bwd dA=dC B^T alone": (fl, lambda q: eng.repeat_gemm(q, dc, b, da, trans_b=True)),
            "bwd dB=A^T dC alone": (fl, lambda q: eng.repeat_gemm(q, a, dc, db, trans_a=True)),
        }
        sec = {k: timer.median_batch(f, reps, warm) for k, (_, f) in modes.items()}
        total = sec["fwd C=AB"] + sec["bwd dA and dB (one call)"]
        out[f"gemm_{n}^3"] = {
            "fwd+bwd_tflops": round(3 * fl / total / 1e12, 2),
            "fwd+bwd_frac_of_mfma_peak": round(3 * fl / total / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
            "fwd+bwd_us": round(total * 1e6, 3),
            "per_mode": {k: roofline(k, "mfma", modes[k][0], v) for k, v in sec.items()}}
        del a, b, dc, c, da, db
    # cfg 4: bandwidth-bound kernels at their configured sizes.
    bw = {}
    r = torch.Generator(device="cuda").manual_seed(4)
    logits = torch.randn(8192, 32000, device="cuda", generator=r) * 2
    tg = torch.randint(0, 32000, (8192,), device="cuda", dtype=torch.int32, generator=r)
    one = torch.ones(1, device="cuda")
    dl = torch.empty_like(logits)
    sec = timer.time(lambda: hip.softmax_xent_backward(logits, tg, one, dl), 20, 3)
    bw["softmax_xent_backward 8192x32000"] = roofline("softmax_xent_backward", "hbm",
                                                     8 * logits.numel() + 4 * 8192, sec)
    del logits, dl
    n = 1 << 28
    x = torch.randn(n, device="cuda", generator=r)
    g = torch.randn(n, device="cuda", generator=r)
    dx = torch.empty(n, device="cuda")
    sec = timer.time(lambda: hip.relu_backward(x, g, dx), 20, 3)
    bw["relu_backward 2^28"] = roofline("relu_backward", "hbm", 12 * n, sec)
    dy = torch.empty(n, device="cuda")
    sec = timer.time(lambda: hip.add_backward(g, dx, dy, False, False), 20, 3)
    bw["add_backward 2^28 (initialise)"] = roofline("add_backward", "hbm", 12 * n, sec)
    sec = timer.time(lambda: hip.add_backward(g, dx, dy, True, True), 20, 3)
    bw["add_backward 2^28 (accumulate)"] = roofline("add_backward", "hbm", 20 * n, sec)
    del dy
    m = torch.zeros(n, device="cuda")
    v = torch.zeros(n, device="cuda")
    sec = timer.time(lambda: hip.adam(x, g, m, v, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0.1, 0.001), 20, 3)
    bw["adam 2^28"] = roofline("adam", "hbm", 28 * n, sec)
    del x, g, dx, m, v
    out["bandwidth_cfg4"] = bw
    torch.cuda.empty_cache()
    log("bench: wide Conv2d layers, implicit GEMM")
    out["conv_wide_implicit_gemm"] = conv_wide_leg(hip, timer, torch)
    # The other bandwidth-bound kernels of the path, at the shapes cfg 5 gives
    # them (16 x 512 tokens, d 1024, FFN 4096, 16 heads of 512 x 512 scores),
    # and max-pool at a large image batch, launched back to back from native
    # code (a ~20 us kernel launched from Python leaves the GPU idle between
    # calls). Bytes are the algorithmic ones: every input read once, every
    # output written once.
    out["bandwidth_transformer_shapes"] = bandwidth_legs(hip, eng, timer, torch, r, 8192, 1024,
                                                         8192, 4096, 16 * 16 * 512, 512,
                                                         (64, 64, 112, 112), 100)
    torch.cuda.empty_cache()
    # The same kernels at cfg 4's size, 2^28 elements, where the launch's ramp
    # and tail are a small part of the time.
    n = 1 << 28
    out["bandwidth_2^28"] = bandwidth_legs(hip, eng, timer, torch, r, n // 1024, 1024, n // 4096,
                                           4096, n // 512, 512, (256, 64, 128, 128), 5)
    torch.cuda.empty_cache()
    return out


def conv_wide_leg(hip, timer, torch):
    """Wide Conv2d layers of ResNet stages through the implicit-GEMM entry points
    (forward; the backward's dx, dW and db in one call) against the explicit im2col
    composition's own kernels (im2col + product; dcols product + col2im + dW product,
    without its bias, permute and copies, so a lower bound on what it costs). FLOPs are
    2 N oH oW C kH kW C_out per product."""
    legs = {}
    for shape, co, k, s, p in [((32, 128, 28, 28), 128, 3, 1, 1), ((16, 64, 56, 56), 128, 3, 2, 1),
                               ((32, 256, 14, 14), 256, 3, 1, 1)]:
        n, c, h, w = shape
        r = torch.Generator(device="cuda").manual_seed(c + co)
        x = torch.randn(shape, device="cuda", generator=r)
        wt = torch.randn(co, c, k, k, device="cuda", generator=r) * 0.05
        b = torch.randn(co, device="cuda", generator=r)
        oh = (h + 2 * p - k) // s + 1
        g = torch.randn(n, co, oh, oh, device="cuda", generator=r)
        kk, pix = c * k * k, oh * oh
        fl = 2.0 * n * pix * kk * co
        fwd = timer.time(lambda: hip.conv2d_igemm(x, wt, b, s, p), 20, 3)
        bwd = timer.time(lambda: hip.conv2d_igemm_backward(x, wt, g, s, p), 20, 3)
        w2 = wt.reshape(co, kk)
        g2 = g.reshape(n, co, pix).permute(0, 2, 1).contiguous().reshape(n * pix, co)
        cols = hip.im2col(x, k, k, s, p)
        cfwd = timer.time(lambda: hip.gemm(hip.im2col(x, k, k, s, p), w2, trans_b=True), 20, 3)
        cbwd = timer.time(lambda: (hip.col2im(hip.gemm(g2, w2), shape, k, k, s, p),
                                   hip.gemm(g2, cols, trans_a=True)), 20, 3)
        legs[f"{n}x{c}x{h}x{w} -> {co} k{k} s{s} p{p}"] = {
            "forward": roofline("conv2d_igemm", "mfma", fl, fwd),
            "backward (dx, dW, db)": roofline("conv2d_igemm_backward", "mfma", 2 * fl, bwd),
            "im2col_composition_us": {"forward": round(cfwd * 1e6, 2),
                                      "backward": round(cbwd * 1e6, 2)},
            "speedup_over_composition": round((cfwd + cbwd) / (fwd + bwd), 2)}
        del x, wt, b, g, g2, cols
    torch.cuda.empty_cache()
    return legs


def kernel_only(eng, hip, timer, torch):
    """For counter runs: the dominant kernel's leg (the six weight-gradient products of a
    cfg 5 block, launched as in dominant_kernel), the cfg 2 step's dominant launch pair
    (cnn_dominant_kernel), LayerNorm forward and the engine's LayerNorm backward row kernel
    at cfg 5's 8192 x 1024 (100 launches each), then 100 launches of the
    gradient-initialise kernel over 16 Mi floats (reads 64 MiB, writes 64 MiB), the copy of
    known size that scales FETCH_SIZE / WRITE_SIZE to bytes."""
    import ctypes
    roof = dominant_kernel(eng, timer, torch)
    cnn = cnn_dominant_kernel(eng, hip, timer, torch)
    r = torch.Generator(device="cuda").manual_seed(8)
    rows, d = 8192, 1024
    x = torch.randn(rows, d, device="cuda", generator=r)
    gam, bet = torch.randn(d, device="cuda", generator=r), torch.randn(d, device="cuda", generator=r)
    y, xh, inv = hip.layernorm(x, gam, bet)
    ln = timer.time_batch(lambda q: eng.repeat_bandwidth(q, "layernorm", [x, gam, bet, y, xh, inv],
                                                         (rows, d), 1e-5), 100, 3)
    groups = ctypes.c_int64(0)
    part = torch.empty(hip.lib.ehip_layernorm_backward_partials(rows, d, ctypes.byref(groups)),
                       device="cuda")
    dx = torch.empty_like(x)
    lnb = timer.time_batch(lambda q: eng.repeat_bandwidth(
        q, "layernorm_backward_rows", [x, xh, gam, inv, dx, part], (rows, d, groups.value)),
        100, 3)
    del x, y, xh, inv, dx, part
    n = 1 << 24
    src = torch.randn(n, device="cuda")
    dst = torch.empty(n, device="cuda")
    sec = timer.time(lambda: hip.accumulate_grad(dst, src, True), 100, 0)
    print(json.dumps({"dominant": roof, "cnn_dominant": cnn,
                      "layernorm_8192x1024_us": round(ln * 1e6, 3),
                      "layernorm_backward_rows_8192x1024_us": round(lnb * 1e6, 3),
                      "copy_64MiB_us": round(sec * 1e6, 3)}), flush=True)


def _r(v, n=3):
    return None if v is None else round(v, n)


def compact_roof(r, keep_kernel=False):
    out = {"bound": r["bound"], "achieved": r["achieved"], "peak": r["peak"], "unit": r["unit"],
           "frac": r["frac"], "traffic": r["traffic"]}
    if keep_kernel:
        out["kernel"] = r["kernel"]
    return out


def compact(line):
    """The printed line, compacted so that the whole of it survives a log tail of a few KB:
    every leg keeps its rate, roofline fraction and CPU baseline; per-mode and per-shape
    details go to --full-out."""
    roof = dict(compact_roof(line["roofline"], keep_kernel=True))
    roof["us_per_launch"] = line["roofline"]["us_per_launch"]
    roof["flop_per_launch"] = line["roofline"]["flop_per_launch"]
    roof["shapes_tflops"] = {k: v["tflops"] for k, v in line["roofline"]["shapes"].items()}
    if "leg" in line["roofline"]:
        roof["leg"] = line["roofline"]["leg"]
    out = dict(line, roofline=roof)
    ex = line.get("extra")
    if not ex:
        return out
    c = {}
    cnn = ex["cnn_cfg2"]
    c["cnn_cfg2"] = {"steps_per_s": cnn["steps_per_s"], "ms_per_step": cnn["ms_per_step"],
                     "graph_steps_per_s": cnn["graph"]["steps_per_s"],
                     "roofline": dict(compact_roof(cnn["roofline"]),
                                      kernel="conv2 block backward (conv3_pool_backward + "
                                             "conv_weight_reduce)"),
                     "cpu_steps_per_s": cnn.get("cpu_baseline", {}).get("value"),
                     "gpu_over_cpu": cnn.get("gpu_over_cpu")}
    lm = ex["charlm_cfg3"]
    c["charlm_cfg3"] = {"steps_per_s": lm["steps_per_s"], "ms_per_step": lm["ms_per_step"],
                        "achieved_tflops": lm["achieved_tflops"],
                        "frac_of_mfma_peak": lm["frac_of_mfma_peak"],
                        "graph_steps_per_s": lm["graph"]["steps_per_s"],
                        "cpu_steps_per_s": lm.get("cpu_baseline", {}).get("value"),
                        "gpu_over_cpu": lm.get("gpu_over_cpu")}
    for n in (512, 4096):
        g = ex[f"gemm_{n}^3"]
        pm = g["per_mode"]
        c[f"gemm_{n}^3"] = {"fwd+bwd_tflops": g["fwd+bwd_tflops"],
                            "frac": g["fwd+bwd_frac_of_mfma_peak"],
                            "fwd_us": pm["fwd C=AB"]["us_per_launch"],
                            "bwd_us": pm["bwd dA and dB (one call)"]["us_per_launch"]}
    for key in ("bandwidth_cfg4", "bandwidth_transformer_shapes", "bandwidth_2^28"):
        c[key] = {k: [round(v["achieved"]), v["frac"]] for k, v in ex[key].items()}
    c["bandwidth_units"] = "[GB/s, fraction of 8000 GB/s]"
    c["conv_wide_implicit_gemm"] = {
        k: {"fwd_tflops": v["forward"]["achieved"],
            "bwd_tflops": v["backward (dx, dW, db)"]["achieved"],
            "x_composition": v["speedup_over_composition"]}
        for k, v in ex["conv_wide_implicit_gemm"].items()}
    out["extra"] = c
    return out


def step_kernels(db_path, top=40):
    """Per-step kernel table from a rocprofv3 rocpd database (for the kernel profiles): the
    trace is cut into steps after each Adam launch (`adam_multi*`), steps that initialise
    state (ten or more fills) are dropped with five more at each end, and each kernel's
    launches and execution time are averaged per step."""
    import collections
    import re
    import sqlite3
    rows = sqlite3.connect(db_path).execute(
        "select name, duration, grid_x, grid_y, grid_z from kernels order by start").fetchall()
    steps, cur = [], []
    for r in rows:
        cur.append(r)
        if "adam_multi" in r[0]:
            steps.append(cur)
            cur = []
    sel = [s for s in steps if sum("Fill" in k[0] for k in s) < 10][5:-5]
    if not sel:
        print("no steps found")
        return
    agg = collections.defaultdict(lambda: [0, 0.0, None])
    for st in sel:
        for k in st:
            n = re.sub(r"ehip::|\(anonymous namespace\)::|gemm_detail::", "", k[0])[:80]
            agg[n][0] += 1
            agg[n][1] += k[1]
            agg[n][2] = k[2:5]
    ns = len(sel)
    print(f"steps {ns} launches {sum(v[0] for v in agg.values()) / ns:.1f} "
          f"kernel {sum(v[1] for v in agg.values()) / ns / 1e3:.1f} us")
    for n, (c, t, grid) in sorted(agg.items(), key=lambda x: -x[1][1])[:top]:
        print(f"  {c / ns:5.1f} x {t / c / 1e3:7.2f} us = {t / ns / 1e3:6.1f} us  {grid} {n}")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target length of the cfg 2 / cfg 3 reference CPU samples")
    ap.add_argument("--cpu-sample-batch", type=int, default=16,
                    help="sequences of the cfg 5 batch in the reference CPU sample (16: one "
                         "whole step, timed as it is)")
    ap.add_argument("--full-out", default=None,
                    help="also write the uncompacted record (every leg's details) to this file")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the dominant kernel and a copy kernel of known size (for "
                         "rocprofv3 --pmc runs) and print their timings")
    ap.add_argument("--transformer-only", action="store_true",
                    help="the cfg 5 step and its dominant kernel only (no CPU baseline, no "
                         "other configurations): the kernel profile's command")
    ap.add_argument("--step-kernels", default=None, metavar="DB",
                    help="print the per-step kernel table of a rocprofv3 rocpd database (no GPU)")
    ap.add_argument("--charlm-only", action="store_true",
                    help="the cfg 3 char-Transformer leg only (no CPU baseline), printed as "
                         "JSON: the cfg 3 kernel profile's command")
    args = ap.parse_args()
    if args.step_kernels:
        step_kernels(args.step_kernels)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        sys.exit(2)
    if args.transformer_only:
        args.no_cpu = args.no_extra = True

    import torch
    assert torch.cuda.is_available(), "bench.py needs the GPU"
    import engine_capi
    import ehip
    hip = ehip.Backend()
    eng = engine_capi.Engine()
    timer = Timer(torch)

    if args.kernel_only:
        kernel_only(eng, hip, timer, torch)
        return
    if args.charlm_only:
        log("bench: cfg3 char-Transformer training step")
        print(json.dumps(charlm_leg(engine_capi, eng, timer, 0.0)), flush=True)
        return

    log("bench: cfg5 Transformer training step")
    rec = cfg5_leg(engine_capi, eng, timer, args.steps, args.warmup, hip)
    sec = rec["seconds"]
    log(f"bench: {sec * 1e3:.3f} ms/step (median {rec['median_s'] * 1e3:.3f}), "
        f"loss {rec['loss_first_step']:.5f} -> {rec['loss_last']:.5f}")
    log("bench: dominant kernel (cfg5 weight-gradient products)")
    roof = in_step_roofline(rec["dw_probe"], dominant_kernel(eng, timer, torch))
    cpu = None
    if not args.no_cpu:
        log("bench: reference CPU baseline (cfg5 sample)")
        cpu = cpu_cfg5_baseline(args.cpu_sample_batch)
        cpu["matmul_512^3"] = cpu_matmul_threads([1, cpu["cores"]])
    extra = None
    if not args.no_extra:
        log("bench: other configurations")
        extra = extras(hip, eng, engine_capi, timer, torch,
                       0.0 if args.no_cpu else args.cpu_seconds)
    info = hip.device_info()
    fl = rec["step_tflop"] * 1e12
    line = {
        "metric": metric_name(),
        "value": round(1.0 / sec, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "cfg5: scaled Transformer LM training step (12 pre-LN blocks, "
                               "d_model 1024, 16 heads, FFN 4096, seq 512, byte vocab 256, "
                               "causal; forward + backward + Adam lr 1e-3), fp32, resident "
                               "batch of random token ids, seeded reference-style init",
                   "global_batch": 16, "seq_len": 512, "parallelism": "single GPU"},
        "median_ms_per_step": round(rec["median_s"] * 1e3, 3),
        "step_tflop": round(rec["step_tflop"], 4),
        "achieved_tflops": round(fl / sec / 1e12, 2),
        "frac_of_mfma_peak": round(fl / sec / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "params": rec["params"],
        "loss_first_step": round(rec["loss_first_step"], 5),
        "loss_last": round(rec["loss_last"], 5),
        "roofline": roof,
        "cpu_baseline": cpu,
        "gpu_over_cpu": None if cpu is None else round((1.0 / sec) / cpu["value"], 1),
        "device": {"name": info.name.decode(), "arch": info.arch.decode(),
                   "compute_units": info.compute_units},
        "extra": extra,
    }
    if args.full_out:
        with open(args.full_out, "w") as f:
            json.dump(line, f)
    print(json.dumps(compact(line)), flush=True)


if __name__ == "__main__":
    main()
