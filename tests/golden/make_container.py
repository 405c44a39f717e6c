"""Writes a small .aff container through the reference's own AffWriter (src/format/aff_writer.cpp,
compiled from the reference sources by oracle/Makefile into oracle/_ref/libaffref.so), for the
container tests. Not a committed fixture: the file is some megabytes, so the tests write it into a
temporary directory whenever the reference build is present.

    python tests/golden/make_container.py OUT.aff

The experts hold arbitrary planes (random code and field bytes, bf16 row scales in [4e-4, 2e-3)),
which exercise every field value; the codebook is the config-1 one the reference fitted."""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))


def write_small_container(path: str, n_layers: int = 2, n_experts: int = 3, hidden: int = 1024,
                          inter: int = 1024, seed: int = 8):
    """Returns (experts uint8 [n_layers][n_experts][stride] in container layout, codebook)."""
    from gpu_util import random_expert_container
    from oracle import load_oracle, load_ref
    O, R = load_oracle(), load_ref()
    lay = O.expert_layout(hidden, inter)
    rng = np.random.default_rng(seed)
    ex = np.stack([np.stack([random_expert_container(rng, hidden, inter, lay) for _ in range(n_experts)])
                   for _ in range(n_layers)])
    cb = np.fromfile(os.path.join(HERE, "c1_codebook.bin"), dtype="<u4")
    meta = json.dumps({"model": "synthetic", "hidden_size": hidden, "moe_intermediate_size": inter,
                       "n_routed_experts": n_experts, "num_experts_per_tok": 2})
    R.write_container(path, meta, ex, cb, hidden, inter)
    return ex, cb


if __name__ == "__main__":
    write_small_container(sys.argv[1])
    print("written", sys.argv[1])
