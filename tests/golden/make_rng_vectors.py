"""Writes tests/golden/rng_vectors.npz: outputs of the reference's own Drop generators
(src/tkm_gpu.cu:751-794: rng_init, rng_u32 and rng_uniform of its four TkmRngType generators),
run on the GPU by oracle/_ref/libref_rng.so (`make -C oracle rng` in the build container builds
it from the reference's text and oracle/ref_rng_harness.hip).

Run on an MI355X box:  python tests/golden/make_rng_vectors.py <out.npz>
The streams: seeds 0, 1, the Drop seeds the runtime derives from its first step seed
(0x13579BDF ^ (node*19937 + 1)) and arbitrary 32-bit values, each with stream indices
0, 1, 2, a few large ones and the top of the range; 16 draws per stream.
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
DRAWS = 16


def streams():
    seeds = [0, 1, 0xFFFFFFFF, 0x13579BDF] + [0x13579BDF ^ (n * 19937 + 1) for n in (17, 32, 50)] + \
            [0x9E3779B9, 0x7F4A7C15 ^ 0x9E3779B9, 0xDEADBEEF]
    idxs = [0, 1, 2, 511, 4096, 123457, 0x7FFFFFFF, 0xFFFFFFFF]
    s, i = np.meshgrid(np.array(seeds, np.uint32), np.array(idxs, np.uint32), indexing="ij")
    return s.ravel().copy(), i.ravel().copy()


def main(out: str) -> None:
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libref_rng.so"))
    p = ctypes.c_void_p
    lib.ref_rng_run.argtypes = [ctypes.c_int, p, p, ctypes.c_int, ctypes.c_int, p, p]
    seeds, idxs = streams()
    n = seeds.size
    res = {"seeds": seeds, "idxs": idxs}
    for t in (1, 2, 3, 4):
        u32 = np.zeros((n, DRAWS), np.uint32)
        uni = np.zeros((n, DRAWS), np.float32)
        rc = lib.ref_rng_run(t, seeds.ctypes.data, idxs.ctypes.data, n, DRAWS, u32.ctypes.data, uni.ctypes.data)
        assert rc == 0, (t, rc)
        res[f"u32_{t}"] = u32
        res[f"uni_{t}"] = uni
    np.savez(out, **res)
    print(f"wrote {out}: {n} streams x {DRAWS} draws for generators 1-4")


if __name__ == "__main__":
    main(sys.argv[1])
