"""Writes the committed fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

config0_sha256.json  SHA-256 of every tensor of the seeded config-0 problem
                     (K=2048, N=1408, 2-bit, g=128, r=64, M=1, seed 0), which
                     pins the generator's draw order and the packing.
small_linear.npz     a small seeded problem (K=256, N=48, 2-bit, r=32, M=2,
                     seed 123): its packed codes and the exact fp64 output of
                     the fp16-dequantized layer.
"""

import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from glorcq_amd import format as fmt  # noqa: E402
from oracle import glorcq_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def main():
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=0)
    with open(os.path.join(HERE, "config0_sha256.json"), "w") as f:
        json.dump({"codes": sha(p.codes), "scales": sha(p.scales), "zeros": sha(p.zeros),
                   "U": sha(p.U), "SV": sha(p.SV), "x": sha(p.x)}, f, indent=1)
    K, N, bits, rank, M, seed = 256, 48, 2, 32, 2, 123
    s = fmt.make_linear(K, N, bits=bits, rank=rank, M=M, seed=seed)
    y64 = O.linear_forward_fp64(s.x, s.q, s.scales, s.zeros, 128, U=s.U, SV=s.SV)
    np.savez(os.path.join(HERE, "small_linear.npz"), K=K, N=N, bits=bits, rank=rank, M=M,
             seed=seed, codes=s.codes.numpy(), y64=y64.numpy())


if __name__ == "__main__":
    main()
