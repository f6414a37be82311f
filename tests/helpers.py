"""Shared test utilities: tolerances, fixtures writing weights directories."""
import os
import tempfile

import numpy as np
import torch

from bindcraft2_amd import params as bparams

# bf16-level tolerances (north star: max relative error <= 2e-2 on
# activations, gradient cosine >= 0.999).  "max relative error" is taken
# normwise -- max|d| / max|ref| -- and relL2 = ||d|| / ||ref||, because the
# elementwise ratio is ill-conditioned at zero crossings.
ACT_TOL = 2e-2
GRAD_COS = 0.999


def metrics(got, ref):
    got = torch.as_tensor(got, dtype=torch.float64).flatten()
    ref = torch.as_tensor(ref, dtype=torch.float64).flatten()
    d = got - ref
    rel_l2 = (d.norm() / ref.norm().clamp_min(1e-30)).item()
    max_rel = (d.abs().max() / ref.abs().max().clamp_min(1e-30)).item()
    cos = (torch.dot(got, ref) / (got.norm() * ref.norm()).clamp_min(1e-30)).item()
    return {"rel_l2": rel_l2, "max_rel": max_rel, "cos": cos}


def assert_act(got, ref, tol=ACT_TOL, what=""):
    m = metrics(got, ref)
    assert m["rel_l2"] <= tol and m["max_rel"] <= tol, f"{what} {m}"
    return m


def assert_grad(got, ref, cos=GRAD_COS, what=""):
    m = metrics(got, ref)
    assert m["cos"] >= cos, f"{what} {m}"
    return m


def weights_dir(params, tag):
    d = os.path.join(tempfile.gettempdir(), f"bc2n_test_{tag}_{os.getpid()}")
    bparams.write_manifest(d, params)
    return d


def random_mask(n, frac, rng):
    """Pair mask m_i*m_j with a random `frac` of residues zeroed."""
    m = np.ones(n, np.float32)
    k = int(round(frac * n))
    if k:
        m[rng.choice(n, k, replace=False)] = 0.0
    return np.outer(m, m).astype(np.float32), m
