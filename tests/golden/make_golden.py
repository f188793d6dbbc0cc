"""Writes the golden relaxation fixtures in this folder.

The reference ships no vector files for this path, so the fixtures are made
here by an independent statement of its equations: torch autograd of the free
energy in float64 (tests/autograd_ref.py), which shares no code with the C
oracle or the HIP library.  Inputs are float32 values; outputs are float64.

Cases follow the reference's own hot-path tests where it has them:
  bpf_tanh       [6,10,4] tanh, eta 0.1, 5 inputs U(-1,1), T=15
                 (BatchedPcForwardTests.cs:44-72)
  bpf_ffg        the same net with the FFG warm start, T=10 (:74-92)
  <act>_small    [9,8,5] for every activation, biases, T=8
  gelu_reg_prec  [12,9,7,3] GELU, activity regularisation 0.01 and
                 per-layer precisions, T=12

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.autograd_ref import autograd_relax  # noqa: E402
from tests.netgen import make_inputs, make_net  # noqa: E402

CASES = {
    "bpf_tanh": dict(sizes=[6, 10, 4], act="tanh", eta=0.1, T=15, B=5, seed=0, xseed=3, xdist="uniform11",
                     bias=0.1),
    "bpf_ffg": dict(sizes=[6, 10, 4], act="tanh", eta=0.1, T=10, B=4, seed=1, xseed=5, xdist="uniform11",
                    bias=0.1, ffg=True),
    "gelu_reg_prec": dict(sizes=[12, 9, 7, 3], act="gelu", eta=0.1, T=12, B=6, seed=4, xseed=6, xdist="normal",
                          bias=0.2, act_reg=0.01, prec=[1.0, 0.7, 1.3, 1.0]),
}
for _i, _act in enumerate(["linear", "tanh", "relu", "sigmoid", "gelu"]):
    CASES[f"{_act}_small"] = dict(sizes=[9, 8, 5], act=_act, eta=0.1, T=8, B=4, seed=10 + _i, xseed=20 + _i,
                                  xdist="normal", bias=0.2)


def make(name, c):
    W, b, P = make_net(c["sizes"], seed=c["seed"], bias_scale=c["bias"], precisions=c.get("prec"))
    x = make_inputs(c["B"], c["sizes"][0], seed=c["xseed"], dist=c["xdist"])
    top, states, energy = autograd_relax(c["sizes"], c["act"], c["eta"], W, b, P, x, c["T"],
                                         act_reg=c.get("act_reg", 0.0), ffg=c.get("ffg", False))
    arrays = {"sizes": np.asarray(c["sizes"], np.int32), "act": np.asarray(c["act"]),
              "eta": np.float64(c["eta"]), "act_reg": np.float64(c.get("act_reg", 0.0)),
              "ffg": np.int32(bool(c.get("ffg", False))), "steps": np.int32(c["T"]),
              "precisions": np.asarray(P, np.float32), "x": x, "top": top, "energy": energy}
    for l, (w, bb) in enumerate(zip(W, b), start=1):
        arrays[f"W{l}"] = w
        arrays[f"b{l}"] = bb
    for l, s in enumerate(states):
        arrays[f"state{l}"] = s
    np.savez(os.path.join(HERE, f"{name}.npz"), **arrays)


def load(path):
    """A fixture as a dict (numpy only, no pickles)."""
    z = np.load(path, allow_pickle=False)
    L = len(z["sizes"])
    return {"name": os.path.basename(path)[:-4], "sizes": [int(s) for s in z["sizes"]], "act": str(z["act"]),
            "eta": float(z["eta"]), "act_reg": float(z["act_reg"]), "ffg": bool(z["ffg"]),
            "steps": int(z["steps"]), "precisions": z["precisions"], "x": z["x"],
            "W": [z[f"W{l}"] for l in range(1, L)], "b": [z[f"b{l}"] for l in range(1, L)],
            "top": z["top"], "energy": z["energy"], "states": [z[f"state{l}"] for l in range(L)]}


def fixtures():
    return sorted(os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith(".npz"))


if __name__ == "__main__":
    for n, c in CASES.items():
        make(n, c)
        print("wrote", n)
