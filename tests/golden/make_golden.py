"""Writes the golden fixtures under tests/golden/.

philox4x64_10.json: raw Philox4x64-10 blocks taken from numpy.random.Philox
(numpy's bit generator is Philox4x64-10 and increments its 256-bit counter
before producing each block, so the block for counter c is read from a
generator started at c-1).  Run:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def philox_cases():
    rng = np.random.default_rng(20260101)
    cases = []
    specials = [([0, 0, 0, 0], [0, 0]), ([M64] * 4, [M64, M64]), ([1, 0, 0, 0], [0, 0]),
                ([0, 7, 0, 0], [42, 0])]
    for ctr, key in specials:
        cases.append((ctr, key))
    for _ in range(12):
        ctr = [int(x) for x in rng.integers(0, 2**63, 4, dtype=np.uint64)]
        key = [int(x) for x in rng.integers(0, 2**63, 2, dtype=np.uint64)]
        cases.append((ctr, key))
    out = []
    for ctr, key in cases:
        c = sum(v << (64 * i) for i, v in enumerate(ctr))
        cm1 = (c - 1) % (1 << 256)
        start = [(cm1 >> (64 * i)) & M64 for i in range(4)]
        bg = np.random.Philox(key=np.array(key, dtype=np.uint64),
                              counter=np.array(start, dtype=np.uint64))
        out.append({"ctr": ctr, "key": key, "out": [int(x) for x in bg.random_raw(4)]})
    return out


def main():
    with open(os.path.join(HERE, "philox4x64_10.json"), "w") as f:
        json.dump({"source": "numpy.random.Philox " + np.__version__, "cases": philox_cases()}, f,
                  indent=1)


if __name__ == "__main__":
    main()
