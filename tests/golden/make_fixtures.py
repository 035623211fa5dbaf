"""Writes the committed golden fixtures from the f64 oracle.

    python tests/golden/make_fixtures.py

The reference (Rust over Burn) holds no golden vectors and cannot run here, so
these fixtures are the oracle's own f64 outputs on seeded inputs: they pin the
GPU path and guard the oracle against regressions.  The oracle itself is
pinned by the relational/closed-form checks in tests/test_oracle.py.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from inputs import mamba1_inputs, ssd2_inputs  # noqa: E402


def ssd2_small():
    # config 0 distributions, reduced to b=1, L=256 (chunk 64, H8 P64 N64 G1)
    inp = ssd2_inputs(seed=20260, b=1, l=256, h=8, p=64, g=1, n=64, h0=True)
    y, hT = oracle.ssd2(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["h0"],
                        chunk=64, form="serial", prec=64)
    np.savez(os.path.join(HERE, "ssd2_cfg0_small.npz"), chunk=np.int32(64), y=y, final_state=hT,
             **{k: v for k, v in inp.items()})


def mamba1_small():
    # config 2 distributions, reduced to b=1, d=64, L=256, N=16
    inp = mamba1_inputs(seed=20261, b=1, d=64, l=256, n=16, h0=True)
    y, hT = oracle.mamba1_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"], inp["D"],
                               inp["z"], h0=inp["h0"], prec=64)
    np.savez(os.path.join(HERE, "mamba1_cfg2_small.npz"), y=y, final_state=hT, **inp)


if __name__ == "__main__":
    ssd2_small()
    mamba1_small()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
