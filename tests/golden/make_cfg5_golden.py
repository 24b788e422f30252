#!/usr/bin/env python3
"""Writes tests/golden/cfg5_reference.npz: the compiled reference engine (oracle/_ref, built by
oracle/Makefile from the reference's own sources) training the cfg 5 Transformer, twice: as the
reference's Release build compiles it (g++ -O3, no -march, so no FMA contraction), and with
FMA contraction (-mfma -ffp-contract=fast), another valid fp32 rounding of the same code. The
second run measures how far the reference's own results move with rounding alone, which is
the tolerance the GPU test allows per step once the trajectory is past the north-star 1e-5.

Workload: the character model of the reference's
examples/charlm_demo.cpp:57-87 at 12 pre-LN blocks, d_model 1024, 16 heads, FFN 4096,
context 512, byte vocabulary 256, batch 16, causal mask; parameters from
workloads.lm_init_params(seed 11) (the reference initialisers' distributions), tokens and
targets from workloads.lm_inputs(seed 3); STEPS Adam steps at lr 1e-3 on that one batch.

Stored (all arrays, no pickled objects); <v> is "" for the Release build, "_fma" for the
contracted one:
  losses<v>        float32 [STEPS]  the loss of every step (before its update)
  names            str [T]          every parameter tensor, in parameter order
  grad_norms<v>    float64 [T]      L2 norm of each tensor's step-1 gradient
  param_norms<v>   float64 [T]      L2 norm of each tensor after the last step
  update_norms<v>  float64 [T]      L2 norm of each tensor's update (last step minus initial)
  s_<name>_idx     int64            sampled flat indices of a selected tensor (all of it when
                                    it has at most SAMPLE elements)
  s_<name>_g<v>    float32          its step-1 gradient at those indices
  s_<name>_p<v>    float32          its value after the last step at those indices
  meta             str              JSON: workload, seeds, threads, CPU, wall times

A cfg 5 step of the reference takes minutes on a few host cores, far too long for a GPU test,
so the GPU test (tests/test_cfg5_parity.py) compares the engine with these vectors; the
inputs and parameters are regenerated from the seeds on both sides.

Usage: python tests/golden/make_cfg5_golden.py [--steps N] [--threads T]
  Each variant's raw result is kept in --work (resumable); the npz is written at the end.
"""
import argparse
import json
import os
import platform
import sys
import time
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "cpp-ai-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import workloads as W  # noqa: E402

PARAM_SEED, INPUT_SEED, LR = 11, 3, 1e-3
SAMPLE = 4096
SELECTED = ["embedding.weight", "block0.attn.query.weight", "block0.attn.query.bias",
            "block0.ff1.weight", "block0.ff1.bias", "block5.attn.out.weight",
            "block5.norm1.beta", "block11.norm2.gamma", "block11.ff2.weight", "head.weight",
            "head.bias"]


def sample_indices(name, size):
    """All of a small tensor; else SAMPLE distinct indices drawn from a seed fixed by the
    tensor's name (crc32), sorted."""
    if size <= SAMPLE:
        return np.arange(size, dtype=np.int64)
    r = np.random.default_rng(zlib.crc32(name.encode()))
    return np.sort(r.choice(size, SAMPLE, replace=False)).astype(np.int64)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


VARIANTS = {"": "libref_engine.so", "_fma": "libref_engine_fma.so"}


def cache_path(args, suffix):
    return os.path.join(args.work, f"cfg5_ref{suffix}_{args.steps}.npz")


def run_variant(suffix, args, params, ids, targets):
    """One training run of the compiled reference, cached in args.work by variant and steps.
    Each run happens in a child process: the reference's buffer pool keeps every block it
    ever allocated (about 30 GB for this model), so two runs in one process would hold
    both."""
    cache = cache_path(args, suffix)
    if not os.path.exists(cache):
        import subprocess
        subprocess.run([sys.executable, os.path.abspath(__file__), "--steps", str(args.steps),
                        "--threads", str(args.threads), "--work", args.work,
                        "--variant", "fma" if suffix else "release"], check=True)
    with np.load(cache, allow_pickle=False) as z:
        return z["losses"], z["final"], z["g0"], float(z["wall"])


def compute_variant(suffix, args, params, ids, targets):
    from _oracle import Ref
    cache = cache_path(args, suffix)
    b, s, vocab, d, heads, ff, layers = W.TRANSFORMER_CFG5
    ref = Ref(os.path.join(ROOT, "oracle", "_ref", VARIANTS[suffix]))
    ref.set_threads(args.threads)
    assert ref.charlm_num_params(vocab, s, d, heads, ff, layers) == params.size
    t0 = time.time()
    losses, final, g0 = ref.charlm_train(ids, targets, vocab, d, heads, ff, layers, params,
                                         args.steps, LR, grads0=True)
    wall = time.time() - t0
    print(f"reference{suffix or ' (Release)'} cfg5: {args.steps} steps in {wall:.1f} s, "
          f"losses {losses}", flush=True)
    os.makedirs(args.work, exist_ok=True)
    np.savez(cache, losses=losses, final=final, g0=g0, wall=wall)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--out", default=os.path.join(HERE, "cfg5_reference.npz"))
    ap.add_argument("--work", default="/tmp/cfg5_golden")
    ap.add_argument("--variant", choices=["release", "fma"], help=argparse.SUPPRESS)
    args = ap.parse_args()

    b, s, vocab, d, heads, ff, layers = W.TRANSFORMER_CFG5
    params = W.lm_init_params(PARAM_SEED, vocab, d, ff, layers)
    ids, targets = W.lm_inputs(INPUT_SEED, b, s, vocab)
    if args.variant:  # the child process of run_variant
        compute_variant("" if args.variant == "release" else "_fma", args, params, ids, targets)
        return
    layout = W.lm_param_layout(vocab, d, ff, layers)
    out, walls = {}, {}
    names = [name for name, _, _ in layout]
    for suffix in VARIANTS:
        losses, final, g0, wall = run_variant(suffix, args, params, ids, targets)
        walls[suffix or "release"] = round(wall, 1)
        gn, pn, un = [], [], []
        off = 0
        for name, shape, _ in layout:
            n = int(np.prod(shape))
            g, p, p0 = g0[off:off + n], final[off:off + n], params[off:off + n]
            gn.append(np.linalg.norm(g.astype(np.float64)))
            pn.append(np.linalg.norm(p.astype(np.float64)))
            un.append(np.linalg.norm(p.astype(np.float64) - p0.astype(np.float64)))
            if name in SELECTED:
                idx = sample_indices(name, n)
                out[f"s_{name}_idx"] = idx
                out[f"s_{name}_g{suffix}"] = g[idx]
                out[f"s_{name}_p{suffix}"] = p[idx]
            off += n
        assert off == params.size
        out[f"losses{suffix}"] = losses
        out[f"grad_norms{suffix}"] = np.array(gn)
        out[f"param_norms{suffix}"] = np.array(pn)
        out[f"update_norms{suffix}"] = np.array(un)
    meta = {"workload": "cfg5 Transformer: 12 pre-LN blocks, d_model 1024, 16 heads, FFN 4096, "
                        "context 512, vocab 256, batch 16, causal; Adam lr 1e-3",
            "dims": W.TRANSFORMER_CFG5, "param_seed": PARAM_SEED, "input_seed": INPUT_SEED,
            "lr": LR, "steps": args.steps, "threads": args.threads, "cpu": cpu_model(),
            "wall_s": walls, "generator": "tests/golden/make_cfg5_golden.py",
            "reference": "oracle/_ref/libref_engine.so (reference src/*.cpp, g++ -O3, no -march)",
            "reference_fma": "oracle/_ref/libref_engine_fma.so (the same sources, g++ -O3 -mfma "
                             "-ffp-contract=fast)"}
    np.savez_compressed(args.out, names=np.array(names), meta=np.array(json.dumps(meta)), **out)
    print(f"wrote {args.out}", flush=True)


if __name__ == "__main__":
    main()
