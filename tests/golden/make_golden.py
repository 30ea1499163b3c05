"""Writes the golden fixtures of tests/test_golden.py from the CPU oracle.

    python tests/golden/make_golden.py

c1_int8.npz: BASELINE.json config 1 (sp.random(512, 512, density 0.1,
random_state=0), B 512x128 N(0,1) from numpy default_rng(0), INT8 per-tile A,
per-tensor B): the int32 accumulators of A @ B, the row-mean output (sha256
of its bytes and a seeded sample of entries), and sha256 digests of the
quantised inputs so that a change of the input generators is detected.
hand_case.npz: a two-tile row with hand-computable accumulators and row-mean.
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import cases  # noqa: E402
import oracle  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1():
    A, B = cases.c1_plumbing()
    dense = np.asarray(A.todense(), dtype=np.float32)
    tiles, br, bc = oracle.csr_tiles(dense)
    q, s = oracle.quantize_i8_blocks(tiles)
    bq, bs = oracle.quantize_i8_tensor(B)
    Ab = oracle.Bsr(q, s, br, bc, (512, 512))
    acc = oracle.i8_acc(Ab, bq)
    out = oracle.row_mean(Ab, acc, bs)
    idx = np.random.default_rng(0).choice(out.size, 4096, replace=False)
    np.savez_compressed(os.path.join(HERE, "c1_int8.npz"), acc=acc, out_sample_idx=idx,
                        out_sample=out.reshape(-1)[idx], out_sha256=sha(out), tiles_sha256=sha(q),
                        scales_sha256=sha(s), b_sha256=sha(bq), b_scale=np.float32(bs))


def hand():
    q = np.zeros((2, 32, 32), np.int8)
    q[0, 0, 0], q[1, 0, 0], q[0, 5, 7] = 3, 5, -128
    s = np.array([0.5, 0.25], np.float32)
    br, bc = np.array([0, 0], np.int32), np.array([0, 1], np.int32)
    B = np.zeros((64, 4), np.int8)
    B[0, 0], B[32, 0], B[7, 3] = 7, 11, 127
    Ab = oracle.Bsr(q, s, br, bc, (32, 64))
    acc = oracle.i8_acc(Ab, B)
    np.savez_compressed(os.path.join(HERE, "hand_case.npz"), tiles=q, scales=s, block_rows=br,
                        block_cols=bc, b=B, b_scale=np.float32(2.0), acc=acc,
                        row_mean=oracle.row_mean(Ab, acc, np.float32(2.0)))


if __name__ == "__main__":
    c1()
    hand()
    print("fixtures written to", HERE)
