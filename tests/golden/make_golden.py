"""Writes the committed golden fixtures with the CPU checker (run from the repo root: python tests/golden/make_golden.py).

Each fixture stores the generator parameters, the inputs x and the checker's outputs (sel, wts, y and Q8_K(x));
the weights are regenerated from tests/golden/gen.py by whoever reads the fixture.
  block_small.npz  : E = 1024, H = 512, 16 experts, 4 groups / top-2 groups / top-4, 5 tokens
  decode_full.npz  : E = 7168, H = 2048 (DeepSeek-R1 dims), 16 routed experts, 8 groups / top-4 / top-8, 2 tokens
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as orc  # noqa: E402
from tests.golden import gen  # noqa: E402

CASES = {
    "block_small": dict(seed=101, n_exp=16, E=1024, H=512, n=5, n_group=4, topk_group=2, topk=4),
    "decode_full": dict(seed=202, n_exp=16, E=7168, H=2048, n=2, n_group=8, topk_group=4, topk=8),
}


def make(name):
    c = CASES[name]
    W, b, gate, up, down, sh = gen.layer(c["seed"], c["n_exp"], c["E"], c["H"])
    x = gen.uniform(c["seed"], 3, (c["n"], c["E"]), 2.0)
    out = orc.moe_forward(x, W, b, gate, up, down, *sh, n_group=c["n_group"], topk_group=c["topk_group"],
                          topk=c["topk"], H=c["H"])
    q, d, _ = orc.quantize_q8k(x)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), x=x, sel=out["sel"], wts=out["wts"], y=out["y"], xq=q, xd=d,
                        **{k: np.int64(v) for k, v in c.items()})
    print(name, "sel", out["sel"].tolist())


if __name__ == "__main__":
    for n in (sys.argv[1:] or CASES):
        make(n)
