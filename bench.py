#!/usr/bin/env python3
"""Benchmark of the fp32 training path on one MI355X.

Prints ONE JSON line. The headline workload is BASELINE.json's configs[1]: the small CNN
training step (conv 1->8 -> ReLU -> pool, conv 8->16 -> ReLU -> pool, linear 784->10,
softmax cross-entropy, Adam lr 1e-3) on a resident synthetic batch of 64 MNIST-shaped
images. `value` is training steps per second through the C++ engine (forward, backward and
the Adam update, all on the GPU), timed with HIP events on the engine's stream over exactly
--steps steps after --warmup untimed steps.

The same line carries:
  roofline      the step's dominant kernel, timed live in isolation with HIP events at
                its in-step shape, against its roofline (HBM or fp32 MFMA);
  cpu_baseline  the reference engine compiled from its own sources (oracle/_ref), running
                the same training step on the host cores for a bounded sample;
  extra         the other configurations: cfg 1 GEMMs (512^3 and 4096^3), cfg 3 and cfg 5
                training steps, cfg 4 bandwidth kernels, each with its roofline fraction.

Only the cpu_baseline leg touches oracle/ (through tests/_oracle.py), as the reference
being timed; nothing measured on the GPU goes through it.
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

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, published
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def metric_name():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


# ------------------------------------------------------------------ inputs

def cnn_inputs(seed=2, batch=64):
    """Pixels U[0,1], labels U{0..9}, Kaiming-uniform weights, zero biases."""
    r = np.random.default_rng(seed)
    x = r.uniform(0.0, 1.0, (batch, 1, 28, 28)).astype(np.float32)
    labels = r.integers(0, 10, batch)
    shapes = [(8, 1, 3, 3), (8,), (16, 8, 3, 3), (16,), (784, 10), (1, 10)]
    params = []
    for shp in shapes:
        n = int(np.prod(shp))
        if len(shp) == 1 or shp[0] == 1:
            params.append(np.zeros(n, np.float32))
        else:
            fan_in = int(np.prod(shp[1:])) if len(shp) == 4 else shp[0]
            lim = np.sqrt(6.0 / fan_in)
            params.append(r.uniform(-lim, lim, n).astype(np.float32))
    return x, labels, np.concatenate(params)


def lm_inputs(seed, batch, seq, vocab):
    r = np.random.default_rng(seed)
    ids = r.integers(0, vocab, (batch, seq)).astype(np.float32)
    targets = r.integers(0, vocab, batch * seq)
    return ids, targets


def lm_step_flops(batch, seq, d, ff, vocab, layers):
    """Algorithmic FLOPs of one training step: every GEMM forward (2mnk) plus its two
    backward products; the full S x S scores are computed (the mask saves nothing)."""
    t = batch * seq
    per_block = 2 * t * d * d * 4 + 2 * t * d * ff * 2 + 2 * batch * seq * seq * d * 2
    fwd = layers * per_block + 2 * t * d * vocab
    return 3 * fwd


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


# ------------------------------------------------------------------ legs

def headline(engine_mod, timer, steps, warmup):
    x, labels, params = cnn_inputs()
    eng = engine_mod.Engine()
    tr = engine_mod.Trainer.cnn(eng, x, labels, params, lr=1e-3)
    first = None
    for i in range(2):
        tr.step()
        if i == 0:
            first = tr.loss()
    sec = timer.time(tr.step, steps, warmup)
    last = tr.loss()
    assert np.isfinite(first) and np.isfinite(last), (first, last)
    tr.close()
    return sec, first, last


def dominant_kernel(eng, hip, timer, torch):
    """The CNN step's largest kernel by total time (rocprofv3 --kernel-trace --stats of
    this benchmark, profiles/cnn_step_kernels.md): the backward of the fused conv2 block
    (Conv2d 8 -> 16, 3x3, pad 1 -> ReLU -> MaxPool2d 2 on a 64 x 8 x 14 x 14 input) --
    conv3_pool_backward (per tile of four rows: the output gradient scattered from the
    pooled cells into LDS, the input gradient and the weight-gradient partials in one
    launch) and conv_weight_reduce (the partials' ordered sum) -- timed as that launch
    pair.
    HBM-bound by its data, latency-bound at this size: algorithmic bytes = x, the pooled
    gradient, the pooled values, the argmax and the weights read once, dx, dW and db
    written once."""
    r = torch.Generator(device="cuda").manual_seed(5)
    x = torch.rand(64, 8, 14, 14, device="cuda", generator=r)
    w = torch.rand(16, 8, 3, 3, device="cuda", generator=r) * 0.6 - 0.3
    b = torch.zeros(16, device="cuda")
    out, am = hip.conv2d_relu_maxpool(x, w, b, 1, 1, 2)
    g = torch.randn(out.shape, device="cuda", generator=r)
    dx, dw, db = torch.empty_like(x), torch.empty_like(w), torch.empty_like(b)
    cw, pw = hip.conv_relu_pool_windows(x.shape, w.shape, 1, 1, 2)
    sec = timer.time_batch(
        lambda n: eng.repeat_conv_relu_pool_backward(n, x, w, g, out, am, dw, db, cw, pw, dx=dx),
        500, 50)
    work = 4 * (2 * x.numel() + 3 * out.numel() + 2 * w.numel() + b.numel())
    return roofline("conv3_pool_backward<2,4,512>+conv_weight_reduce (conv2 block dx/dW/db, "
                    "64x8x14x14, 16 filters 3x3, pool 2)", "hbm", work, sec,
                    committed_traffic("conv2_block_backward"))


def kernel_only(eng, hip, timer, torch):
    """For counter runs: 100 launches of the dominant kernel, then 100 launches of the
    gradient-initialise kernel over 16 Mi floats (reads 64 MiB, writes 64 MiB), the copy
    of known size that scales FETCH_SIZE / WRITE_SIZE to bytes."""
    roof = dominant_kernel(eng, hip, timer, torch)
    n = 1 << 24
    src = torch.randn(n, device="cuda")
    dst = torch.empty(n, device="cuda")
    sec = timer.time(lambda: hip.accumulate_grad(dst, src, True), 100, 0)
    print(json.dumps({"dominant": roof, "copy_64MiB_us": round(sec * 1e6, 3)}), flush=True)


def cpu_baseline(seconds_target):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _oracle import Ref
    x, labels, params = cnn_inputs()
    threads = int(os.environ.get("BENCH_CPU_THREADS", "0")) or min(16, os.cpu_count() or 1)
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
    threads = int(os.environ.get("BENCH_CPU_THREADS", "0")) or min(16, os.cpu_count() or 1)
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


# (batch, seq, vocab, d_model, heads, ffn, layers, timed steps, warm-up steps)
LM_CONFIGS = {"charlm_cfg3": (32, 64, 121, 96, 4, 384, 2, 100, 10),
              "transformer_cfg5": (16, 512, 256, 1024, 16, 4096, 12, 5, 2)}


def lm_leg(engine_mod, eng, timer, dims, keep_params=False):
    """One character-model Transformer training-step measurement (forward +
    backward + Adam on a resident synthetic batch); returns (record, initial
    parameters or None)."""
    b, s, vocab, d, h, ff, layers, steps, warm = dims
    ids, targets = lm_inputs(3, b, s, vocab)
    tr = engine_mod.Trainer.charlm(eng, ids, targets, vocab, d, h, ff, layers, lr=1e-3)
    p0 = tr.params() if keep_params else None
    first = None
    if warm > 0:
        tr.step()
        first = tr.loss()
    sec = timer.time(tr.step, steps, max(warm - 1, 0))
    fl = lm_step_flops(b, s, d, ff, vocab, layers)
    rec = {"steps_per_s": round(1.0 / sec, 3), "ms_per_step": round(sec * 1e3, 3),
           "params": int(tr.num_params()), "step_tflop": round(fl / 1e12, 4),
           "achieved_tflops": round(fl / sec / 1e12, 2),
           "frac_of_mfma_peak": round(fl / sec / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
           "loss_first_step": None if first is None else round(first, 5),
           "loss_after": round(tr.loss(), 5)}
    tr.close()
    return rec, p0


def bandwidth_large(hip, timer, torch, r):
    """LayerNorm forward / backward, the bias-gradient column sum, softmax forward /
    backward and max-pool forward / backward over 2^28-element tensors, with the
    algorithmic bytes of the cfg 5 legs."""
    bl = {}
    n = 1 << 28
    rows, d = n // 1024, 1024
    x = torch.randn(rows, d, device="cuda", generator=r)
    gam = torch.randn(d, device="cuda", generator=r)
    bet = torch.randn(d, device="cuda", generator=r)
    sec = timer.time(lambda: hip.layernorm(x, gam, bet), 20, 3)
    bl[f"layernorm {rows}x{d}"] = roofline("layernorm", "hbm", 12 * n + 4 * rows, sec)
    _, xh, inv = hip.layernorm(x, gam, bet)
    sec = timer.time(lambda: hip.layernorm_backward(x, xh, gam, inv), 20, 3)
    bl[f"layernorm_backward {rows}x{d}"] = roofline("layernorm_backward", "hbm",
                                                    12 * n + 4 * rows + 8 * d, sec)
    del x, xh, inv
    torch.cuda.empty_cache()
    rows, ff = n // 4096, 4096
    gb = torch.randn(rows, ff, device="cuda", generator=r)
    sec = timer.time(lambda: hip.sum_axis(gb, 1, rows, ff), 20, 3)
    bl[f"bias_grad_sum {rows}x{ff}"] = roofline("sum_axis", "hbm", 4 * n + 4 * ff, sec)
    del gb
    sc = torch.randn(n // 512, 512, device="cuda", generator=r)
    sec = timer.time(lambda: hip.softmax(sc), 20, 3)
    bl[f"softmax {n // 512}x512"] = roofline("softmax", "hbm", 8 * n, sec)
    y = hip.softmax(sc)
    sec = timer.time(lambda: hip.softmax_backward(y, sc), 20, 3)
    bl[f"softmax_backward {n // 512}x512"] = roofline("softmax_backward", "hbm", 12 * n, sec)
    del sc, y
    torch.cuda.empty_cache()
    im = torch.randn(256, 64, 128, 128, device="cuda", generator=r)
    pooled, am = hip.maxpool(im, 2, 2)
    sec = timer.time(lambda: hip.maxpool(im, 2, 2, out=(pooled, am)), 20, 3)
    bl["maxpool 256x64x128x128 k2"] = roofline("maxpool", "hbm", 6 * n, sec)
    gp = torch.randn_like(pooled)
    dim = torch.empty_like(im)
    sec = timer.time(lambda: hip.maxpool_backward(am, gp, tuple(im.shape), 2, 2, dx=dim), 20, 3)
    bl["maxpool_backward 256x64x128x128 k2"] = roofline("maxpool_backward", "hbm", 6 * n, sec)
    del im, pooled, am, gp, dim
    return bl


def extras(hip, eng, engine_mod, timer, torch, cpu_seconds=0.0):
    out = {}
    # cfg 1: C = A B and both backward products at 512^3 (805.3 MFLOP per trio), and 4096^3.
    for n in (512, 4096):
        r = torch.Generator(device="cuda").manual_seed(n)
        a = torch.randn(n, n, device="cuda", generator=r)
        b = torch.randn(n, n, device="cuda", generator=r)
        dc = torch.randn(n, n, device="cuda", generator=r)
        c, da, db = (torch.empty(n, n, device="cuda") for _ in range(3))
        fl = 2.0 * n ** 3
        modes = {
            "fwd C=AB": lambda r: eng.repeat_gemm(r, a, b, c),
            "bwd dA=dC B^T": lambda r: eng.repeat_gemm(r, dc, b, da, trans_b=True),
            "bwd dB=A^T dC": lambda r: eng.repeat_gemm(r, a, dc, db, trans_a=True),
        }
        sec = {k: timer.time_batch(f, 20 if n == 4096 else 500, 3 if n == 4096 else 50)
               for k, f in modes.items()}
        total = sum(sec.values())
        out[f"gemm_{n}^3"] = {
            "fwd+bwd_tflops": round(3 * fl / total / 1e12, 2),
            "fwd+bwd_frac_of_mfma_peak": round(3 * fl / total / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
            "per_mode": {k: roofline(k, "mfma", fl, v) for k, v in sec.items()}}
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
    # The other bandwidth-bound kernels of the path, at the shapes cfg 5 gives
    # them (16 x 512 tokens, d 1024, FFN 4096, 16 heads of 512 x 512 scores),
    # and max-pool at a large image batch. Bytes are the algorithmic ones:
    # every input read once, every output written once.
    bt = {}
    rows, d, ff = 8192, 1024, 4096
    x = torch.randn(rows, d, device="cuda", generator=r)
    gam = torch.randn(d, device="cuda", generator=r)
    bet = torch.randn(d, device="cuda", generator=r)
    sec = timer.time(lambda: hip.layernorm(x, gam, bet), 20, 3)
    bt["layernorm 8192x1024"] = roofline("layernorm", "hbm", 12 * x.numel() + 4 * rows, sec)
    _, xh, inv = hip.layernorm(x, gam, bet)
    sec = timer.time(lambda: hip.layernorm_backward(x, xh, gam, inv), 20, 3)
    bt["layernorm_backward 8192x1024"] = roofline("layernorm_backward", "hbm",
                                                  12 * x.numel() + 4 * rows + 8 * d, sec)
    del x, xh, inv
    gb = torch.randn(rows, ff, device="cuda", generator=r)
    sec = timer.time(lambda: hip.sum_axis(gb, 1, rows, ff), 20, 3)
    bt["bias_grad_sum 8192x4096"] = roofline("sum_axis", "hbm", 4 * gb.numel() + 4 * ff, sec)
    del gb
    sc = torch.randn(16 * 16 * 512, 512, device="cuda", generator=r)
    sec = timer.time(lambda: hip.softmax(sc), 20, 3)
    bt["softmax 131072x512"] = roofline("softmax", "hbm", 8 * sc.numel(), sec)
    y = hip.softmax(sc)
    sec = timer.time(lambda: hip.softmax_backward(y, sc), 20, 3)
    bt["softmax_backward 131072x512"] = roofline("softmax_backward", "hbm", 12 * sc.numel(), sec)
    del sc, y
    im = torch.randn(64, 64, 112, 112, device="cuda", generator=r)
    pooled, am = hip.maxpool(im, 2, 2)  # outputs reused by the timed calls
    sec = timer.time(lambda: hip.maxpool(im, 2, 2, out=(pooled, am)), 20, 3)
    bt["maxpool 64x64x112x112 k2"] = roofline("maxpool", "hbm", 6 * im.numel(), sec)
    gp = torch.randn_like(pooled)
    dim = torch.empty_like(im)
    sec = timer.time(lambda: hip.maxpool_backward(am, gp, tuple(im.shape), 2, 2, dx=dim), 20, 3)
    bt["maxpool_backward 64x64x112x112 k2"] = roofline("maxpool_backward", "hbm",
                                                       6 * im.numel(), sec)
    del im, pooled, am, gp, dim
    out["bandwidth_transformer_shapes"] = bt
    torch.cuda.empty_cache()
    # The same kernels at cfg 4's size, 2^28 elements, where the launch's ramp
    # and tail are a small part of the time.
    out["bandwidth_2^28"] = bandwidth_large(hip, timer, torch, r)
    torch.cuda.empty_cache()
    # cfg 3 and cfg 5: Transformer training steps.
    for tag, dims in LM_CONFIGS.items():
        ids, targets = lm_inputs(3, dims[0], dims[1], dims[2])
        out[tag], p0 = lm_leg(engine_mod, eng, timer, dims,
                              keep_params=tag == "charlm_cfg3" and cpu_seconds > 0)
        b, s, vocab, d, h, ff, layers, steps, warm = dims
        if p0 is not None:
            log("bench: reference CPU baseline, cfg3")
            cpu = cpu_charlm_baseline(ids, targets, (vocab, d, h, ff, layers), p0, cpu_seconds)
            out[tag]["cpu_baseline"] = cpu
            out[tag]["gpu_over_cpu"] = round(out[tag]["steps_per_s"] / cpu["value"], 1)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the dominant kernel and a copy kernel of known size (for "
                         "rocprofv3 --pmc runs) and print their timings")
    ap.add_argument("--transformer-only", action="store_true",
                    help="run only the cfg5 Transformer step leg (for kernel profiles) and "
                         "print its record")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        sys.exit(2)

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
    if args.transformer_only:
        rec, _ = lm_leg(engine_capi, eng, timer, LM_CONFIGS["transformer_cfg5"])
        print(json.dumps({"transformer_cfg5": rec}), flush=True)
        return

    log("bench: cfg2 CNN training step")
    sec, first, last = headline(engine_capi, timer, args.steps, args.warmup)
    log(f"bench: {sec * 1e3:.4f} ms/step, loss {first:.5f} -> {last:.5f}")
    log("bench: dominant kernel")
    roof = dominant_kernel(eng, hip, timer, torch)
    cpu = None
    if not args.no_cpu:
        log("bench: reference CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)
    extra = None
    if not args.no_extra:
        log("bench: other configurations")
        extra = extras(hip, eng, engine_capi, timer, torch,
                       0.0 if args.no_cpu else args.cpu_seconds)
    info = hip.device_info()
    line = {
        "metric": metric_name(),
        "value": round(1.0 / sec, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "cfg2: small CNN training step (conv 1->8, ReLU, maxpool2, "
                               "conv 8->16, ReLU, maxpool2, linear 784->10, softmax-CE, Adam "
                               "lr 1e-3), fp32, resident batch", "global_batch": 64,
                   "input": "1x28x28", "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": {"name": info.name.decode(), "arch": info.arch.decode(),
                   "compute_units": info.compute_units},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
