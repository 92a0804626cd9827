"""Pin block_hadamard: golden sign vectors written from the reference's own function
(tests/golden/make_hadamard_golden.py), plus orthonormality, block structure and the
Sylvester pattern. Both the oracle and the product's host copy are checked."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import ref
from starkv_serve.kernels import paged_quant as pq

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "hadamard_signs.json")


def _golden():
    with open(GOLDEN) as f:
        return json.load(f)


def _check_against_blocks(T, entry):
    r = entry["rank"]
    assert T.shape == (r, r)
    covered = np.zeros((r, r), bool)
    for blk in entry["blocks"]:
        a, m = blk["start"], blk["m"]
        if m == 0:
            continue
        signs = np.array([1.0 if c == "+" else -1.0 for c in blk["signs"]])
        H = np.array([[(-1) ** bin(i & j).count("1") for j in range(m)] for i in range(m)], float)
        np.testing.assert_allclose(T[a:a + m, a:a + m], signs[:, None] * H / math.sqrt(m), atol=1e-15)
        covered[a:a + m, a:a + m] = True
    # identity elsewhere
    rest = np.where(covered, 0.0, T)
    np.testing.assert_allclose(rest, np.where(covered, 0.0, np.eye(r)), atol=1e-15)
    assert abs(np.abs(T).sum() - entry["abs_sum"]) < 1e-9


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_golden_sequence_and_fresh(impl):
    g = _golden()
    fn = ref.block_hadamard if impl == "oracle" else (lambda r, n, gen: pq.block_hadamard(r, n, gen).numpy())
    gen = torch.Generator().manual_seed(g["seed"])
    for entry in g["k_sequence"]:  # one generator consumed head by head
        _check_against_blocks(np.asarray(fn(entry["rank"], entry["n_out"], gen)), entry)
    for entry in g["v_fresh"]:     # a fresh generator per projection
        T = np.asarray(fn(entry["rank"], entry["n_out"], torch.Generator().manual_seed(g["seed"])))
        _check_against_blocks(T, entry)


@pytest.mark.parametrize("rank", [1, 2, 3, 5, 16, 20, 48, 64, 100, 1290])
def test_orthonormal_and_fold_identity(rank):
    T = ref.block_hadamard(rank, ref.n_outlier(rank), torch.Generator().manual_seed(5))
    np.testing.assert_allclose(T @ T.T, np.eye(rank), atol=1e-12)
    # the loader's fold: U T T^T VS == U VS (checkpoint.py:97)
    rng = np.random.default_rng(rank)
    U, VS = rng.standard_normal((8, rank)), rng.standard_normal((rank, 5))
    np.testing.assert_allclose((U @ T) @ (T.T @ VS), U @ VS, atol=1e-10)
