"""Write tests/golden/hadamard_signs.json from the reference's own block_hadamard.

block_hadamard's sign vectors come from torch's CPU generator stream
(starkv_serve/kernels/paged_quant.py:50-68) consumed head by head with one fresh
generator per projection seeded with HADAMARD_SEED (starkv_serve/checkpoint.py:96-103,
118-122, 146-148). Nothing but the reference itself fixes those bits, so this script
imports that one function from the read-only reference checkout and records its
output as data. It runs only where the reference is mounted; the committed JSON is
what the tests read.

    python tests/golden/make_hadamard_golden.py [/path/to/reference]
"""
import importlib.util
import json
import math
import os
import sys

import torch

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hadamard_signs.json")

# Ranks chosen to hit: no outlier block (rank < 5), 1-wide blocks (consume no
# randomness), non-power-of-two blocks (identity tail), and realistic sizes.
K_RANKS = [16, 32, 48, 64, 24, 7, 1, 3, 128, 80]
V_RANKS = [32, 64, 1280, 1290]


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _blocks(T, rank, n_out):
    """Per block (start, m, signs): T[a+i, a+j] = s_i * H_ij / sqrt(m), H_i0 = 1."""
    out = []
    for a, n in ((0, n_out), (n_out, rank - n_out)):
        if n <= 1:
            out.append({"start": a, "m": 0, "signs": ""})
            continue
        m = 1 << (n.bit_length() - 1)
        col = T[a:a + m, a] * math.sqrt(m)
        out.append({"start": a, "m": m, "signs": "".join("+" if v > 0 else "-" for v in col.tolist())})
    return out


def main():
    pq = _load(os.path.join(REF, "starkv_serve", "kernels", "paged_quant.py"), "_ref_paged_quant")
    g = torch.Generator().manual_seed(pq.HADAMARD_SEED)
    k = []
    for r in K_RANKS:
        T = pq.block_hadamard(r, pq.n_outlier(r), g)
        k.append({"rank": r, "n_out": pq.n_outlier(r), "blocks": _blocks(T, r, pq.n_outlier(r)),
                  "abs_sum": float(T.abs().sum())})
    v = []
    for r in V_RANKS:
        T = pq.block_hadamard(r, pq.n_outlier(r), torch.Generator().manual_seed(pq.HADAMARD_SEED))
        v.append({"rank": r, "n_out": pq.n_outlier(r), "blocks": _blocks(T, r, pq.n_outlier(r)),
                  "abs_sum": float(T.abs().sum())})
    data = {"seed": pq.HADAMARD_SEED, "torch": torch.__version__,
            "k_sequence": k, "v_fresh": v,
            "source": "starkv_serve/kernels/paged_quant.py:50-68 block_hadamard, one generator for "
                      "the K ranks in order, a fresh generator per V rank"}
    with open(OUT, "w") as f:
        json.dump(data, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
