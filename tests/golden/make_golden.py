"""Writes the committed fixtures under tests/golden/.

  q0_<V>x<R>.npy   the subspace iteration's fixed start, torch.randn(V, R, generator=Generator().manual_seed(0)), exactly
                   as the reference builds it (/root/reference/leapquant/state.py:70, kernels.py:2326); regenerated here
                   with this image's torch (no reference code is imported or run).
  oracle_*.npz     small seeded oracle trajectories (GDN / KDA, W = 16 and 64, two to three windows) so that a later change
                   to the oracle itself is caught: inputs, per-step outputs and the final checkpoint.

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))


def write_q0():
    import torch
    for V, R in ((128, 4), (128, 1), (128, 2), (64, 4), (128, 8), (128, 12), (128, 16)):
        q0 = torch.randn(V, R, generator=torch.Generator().manual_seed(0)).numpy().astype(np.float32)
        np.save(os.path.join(HERE, "q0_%dx%d.npy" % (V, R)), q0)


def write_trajectories():
    from tests.fixtures import make_trajectory, to_bits
    for kda in (False, True):
        for L in (16, 64):
            steps = 2 * L + 3 if L <= 16 else L + 3          # two windows at W = 16, one flush at W = 64
            t = make_trajectory(kda=kda, L=L, steps=steps, seed=7 + L + (100 if kda else 0))
            np.savez_compressed(os.path.join(HERE, "oracle_%s_L%d.npz" % ("kda" if kda else "gdn", L)), **to_bits(t))


if __name__ == "__main__":
    write_q0()
    write_trajectories()
