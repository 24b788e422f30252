#!/usr/bin/env python3
"""Writes a synthetic text corpus for the reference's character-level language model demo
(examples/charlm_demo.cpp), which reads ENGINE_REPO_DIR/docs/{DESIGN,PERFORMANCE,
ENGINEERING,CUDA}.md and ENGINE_REPO_DIR/README.md (charlm_demo.cpp:192-195). The demo is
built with ENGINE_REPO_DIR pointing here, in the git-ignored build folder, so it runs on a
machine without the reference checkout and reads the same text under every engine. No
reference text is copied: the files are seeded random sentences over a fixed list of common
English words, with markdown headings, lists and code spans, about 40 KB each.

Usage: make_corpus.py OUT_DIR"""
import os
import sys

import numpy as np

WORDS = """the a an of to in and or for with on at by from as is are was be been it this that
these those each every some any all no not only also then than when while where which what
who how why because so but if else into onto over under between through across after before
during within without about around again once more most less least very much many few other
same such own new old first last next long short small large high low fast slow early late
good better best simple clear exact whole each per engine tensor graph node edge kernel
device host memory buffer stream launch block thread wave tile matrix vector row column
value gradient loss step batch layer model weight bias input output shape size length width
height channel image pixel token sequence head attention score mask softmax norm mean sum
product train test data set run time cost work path call test check result error bound
order sign scale rate peak share load store read write copy move keep hold free take give
make build find use show see say know need want try start stop end begin open close add
remove change grow fall rise turn hand point part place case way fact word line page note
number count table list file name type field form state level mode plan rule goal reason
idea method system process program function class object module library interface
""".split()
PUNCT = [".", ".", ".", ",", ",", ";", ":", "?", "!"]


def sentence(r):
    n = int(r.integers(4, 16))
    words = [WORDS[int(i)] for i in r.integers(0, len(WORDS), n)]
    if r.random() < 0.1:
        words[int(r.integers(0, n))] = str(int(r.integers(0, 4096)))
    if r.random() < 0.15:
        k = int(r.integers(0, n))
        words[k] = "`" + words[k] + "()`"
    words[0] = words[0].capitalize() if r.random() < 0.7 else "The"
    return " ".join(words) + PUNCT[int(r.integers(0, len(PUNCT)))]


def document(r, title, size):
    out = [f"# {title}", ""]
    while sum(len(x) + 1 for x in out) < size:
        kind = r.random()
        if kind < 0.08:
            out += ["", "## " + " ".join(WORDS[int(i)] for i in r.integers(0, len(WORDS), 3)).title(), ""]
        elif kind < 0.2:
            out += [f"- {sentence(r)}" for _ in range(int(r.integers(2, 5)))]
        elif kind < 0.25:
            cols = [WORDS[int(i)] for i in r.integers(0, len(WORDS), 3)]
            out += ["| " + " | ".join(cols) + " |", "|---|---|---|",
                    "| " + " | ".join(str(int(v)) for v in r.integers(0, 999, 3)) + " |"]
        else:
            out.append(" ".join(sentence(r) for _ in range(int(r.integers(2, 6)))))
        out.append("")
    return "\n".join(out) + "\n"


def main():
    out = sys.argv[1]
    os.makedirs(os.path.join(out, "docs"), exist_ok=True)
    r = np.random.default_rng(2024)
    for name in ("DESIGN", "PERFORMANCE", "ENGINEERING", "CUDA"):
        with open(os.path.join(out, "docs", name + ".md"), "w") as f:
            f.write(document(r, name.title(), 40000))
    with open(os.path.join(out, "README.md"), "w") as f:
        f.write(document(r, "Readme", 20000))


if __name__ == "__main__":
    main()
