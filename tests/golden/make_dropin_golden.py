"""Writes the expected outputs of the drop-in check (tests/golden/dropin/):

  <example>.txt       the reference's example program built against the compiled
                      reference engine (tests/dropin/Makefile, _build/ref), run here on
                      the CPU;
  charlm_demo.fma.txt the character-model demo (200 steps, on the synthetic corpus that
                      make_corpus.py writes) run with the FMA-contracted reference: its
                      losses bound how far the reference's own rounding moves the
                      trajectory (tests/test_dropin.py compares the losses, not the text
                      the model generates);
  <example>.tol.json  the output lines whose numbers are not fixed by the program:
                      "random" for a line that two runs of that same program print
                      differently (an unseeded generator), "rounding" for a line it
                      prints differently when the reference engine is compiled with FMA
                      contraction (_build/ref_fma), another valid fp32 rounding. Lines
                      absent from the file print the same under both.

Run from the repository root after `make -C tests/dropin`."""
import json
import os
import re
import subprocess
import sys

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", ".."))
BUILD = os.path.join(ROOT, "tests", "dropin", "_build")
EXAMPLES = ["autograd_demo", "nn_demo", "cnn_demo", "transformer_demo", "main"]
NUMBER = re.compile(r"[-+]?(?:\d+\.\d*|\.\d+|\d+)(?:[eE][-+]?\d+)?")


ARGS = {"charlm_demo": ["200"]}


def run(exe):
    name = os.path.basename(exe)
    r = subprocess.run([exe] + ARGS.get(name, []), capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        sys.exit(f"{exe}: exit status {r.returncode}\n{r.stderr}")
    return r.stdout


def main():
    out_dir = os.path.join(ROOT, "tests", "golden", "dropin")
    os.makedirs(out_dir, exist_ok=True)
    only = sys.argv[1:]
    first = run(os.path.join(BUILD, "ref", "charlm_demo"))
    if not only or "charlm_demo" in only:
        with open(os.path.join(out_dir, "charlm_demo.txt"), "w") as f:
            f.write(first)
        with open(os.path.join(out_dir, "charlm_demo.fma.txt"), "w") as f:
            f.write(run(os.path.join(BUILD, "ref_fma", "charlm_demo")))
        print("charlm_demo: reference and FMA-reference outputs written")
    for name in EXAMPLES:
        if only and name not in only:
            continue
        first = run(os.path.join(BUILD, "ref", name))
        second = run(os.path.join(BUILD, "ref", name)).splitlines()
        fma = run(os.path.join(BUILD, "ref_fma", name)).splitlines()
        lines = first.splitlines()
        if len(second) != len(lines) or len(fma) != len(lines):
            sys.exit(f"{name}: line counts differ between runs")
        tol = {}
        for n, (a, b, c) in enumerate(zip(lines, second, fma), 1):
            if a != b:
                tol[n] = "random"
            elif a != c:
                tol[n] = "rounding" if NUMBER.sub("#", a) == NUMBER.sub("#", c) else "random"
        with open(os.path.join(out_dir, name + ".txt"), "w") as f:
            f.write(first)
        with open(os.path.join(out_dir, name + ".tol.json"), "w") as f:
            json.dump(tol, f, indent=0)
        print(f"{name}: {len(lines)} lines, {sum(1 for v in tol.values() if v == 'random')} "
              f"random, {sum(1 for v in tol.values() if v == 'rounding')} rounding-sensitive")


if __name__ == "__main__":
    main()
