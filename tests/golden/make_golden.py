"""Writes the committed fixtures of tests/golden from the CPU oracle.

iq3s_synth251_block_dots.npy: exact int32 IQ3_S x Q8_1 block dots of the
reference's synthetic test bytes (chimere-server/src/kernels/fused_gate_up.rs:
386-412: weights byte i = i % 251, Q8_1 blocks with d bits 0x1000, s 0 and
q[j] = j % 5), 16 rows x 2048 columns.  Run from the repo root:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402


def synth251(ncols=2048, nrows=16):
    W = (np.arange(nrows * ncols // 256 * 110) % 251).astype(np.uint8)
    xq = np.zeros(ncols // 32 * 36, np.uint8)
    for b in range(ncols // 32):
        xq[b * 36 + 1] = 0x10
        xq[b * 36 + 4:b * 36 + 36] = np.arange(32) % 5
    return W, xq


if __name__ == "__main__":
    W, xq = synth251()
    np.save(os.path.join(ROOT, "tests", "golden", "iq3s_synth251_block_dots.npy"),
            O.block_dots(O.IQ3_S, W, xq, 2048, 16))
    print("written")
