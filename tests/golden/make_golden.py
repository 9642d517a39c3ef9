"""Writes the golden fixtures under tests/golden/ from the float64 oracle.

The reference has no test vectors of its own, so these fixtures are produced
by this build's oracle (oracle/attention_ref.py) on the synthetic inputs of
femtochat_amd.workloads and committed; tests check that the oracle and the
GPU path reproduce them.

  c1_golden.npz    : the README toy config C1 (D16 H2 Hkv1 T4 B2, window (4,0)).
  slice_golden.npz : a C3-shaped slice (D128, one KV group of 2 heads) at
                     T=48 with a document mask and window (20,0), bf16 inputs.
"""
from pathlib import Path
import sys

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from femtochat_amd import workloads as W  # noqa: E402
from oracle import attention_ref as R  # noqa: E402

HERE = Path(__file__).resolve().parent


def c1():
    wl = W.WORKLOADS["C1"]
    h = W.host_inputs(wl)
    O, l, m = R.forward(h.Q, h.K, h.V, h.window, h.positions)
    dQ, dK, dV = R.backward(h.dO, h.Q, h.K, h.V, O, l, m, h.window, h.positions)
    np.savez_compressed(HERE / "c1_golden.npz", Q=h.Q, K=h.K, V=h.V, dO=h.dO, positions=h.positions,
                        window=np.array(h.window), O=O, l=l, m=m, dQ=dQ, dK=dK, dV=dV)


def slice_fixture():
    wl = W.WORKLOADS["C3"]
    h = W.host_inputs(wl, batch=[0])
    T = 48
    Q, K, V, dO = h.Q[:, :T, :2], h.K[:, :T, :1], h.V[:, :T, :1], h.dO[:, :T, :2]
    pos = np.concatenate([np.arange(5, 5 + 17), np.arange(20), np.arange(11)])[None].astype(np.int32)
    window = (20, 0)
    O, l, m = R.forward(Q, K, V, window, pos)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, window, pos)
    np.savez_compressed(HERE / "slice_golden.npz", Q=Q, K=K, V=V, dO=dO, positions=pos, window=np.array(window),
                        O=O.astype(np.float32), l=l, m=m, dQ=dQ.astype(np.float32), dK=dK.astype(np.float32),
                        dV=dV.astype(np.float32))


if __name__ == "__main__":
    c1()
    slice_fixture()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
