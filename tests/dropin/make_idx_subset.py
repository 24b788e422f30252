#!/usr/bin/env python3
"""Writes a small synthetic data set in the MNIST IDX format for the reference's data-reader
test (its tests/test_nn.cpp, test_idx_reader), which looks for the repository subset's file
names under ENGINE_DATA_DIR/mnist. No reference data is copied: the images are seeded random
bytes with saturated pixels, the labels seeded digits whose first is a 5, as the test expects
of MNIST's first training digit. The IDX layout (big-endian magic 0x00000803 / 0x00000801,
then the dimensions, then unsigned bytes) is the published format the reader parses.

Usage: make_idx_subset.py OUT_DIR"""
import os
import struct
import sys

import numpy as np


def write_images(path, images):
    n, h, w = images.shape
    with open(path, "wb") as f:
        f.write(struct.pack(">IIII", 0x00000803, n, h, w))
        f.write(images.astype(np.uint8).tobytes())


def write_labels(path, labels):
    with open(path, "wb") as f:
        f.write(struct.pack(">II", 0x00000801, len(labels)))
        f.write(labels.astype(np.uint8).tobytes())


def main():
    out = sys.argv[1]
    os.makedirs(out, exist_ok=True)
    r = np.random.default_rng(5)
    for split, n in (("train", 128), ("test", 64)):
        images = r.integers(0, 256, (n, 28, 28))
        images[:, 10:18, 12:16] = 255  # every image has saturated pixels
        labels = r.integers(0, 10, n)
        labels[0] = 5
        write_images(os.path.join(out, f"subset-{split}-images-idx3-ubyte"), images)
        write_labels(os.path.join(out, f"subset-{split}-labels-idx1-ubyte"), labels)


if __name__ == "__main__":
    main()
