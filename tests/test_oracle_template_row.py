"""Pins of the oracle's template row (modules_multimer.py:1080-1137,
all_atom_multimer.py:880-941, geometry/vector.py:187-212): the dihedral
against quadruples built with a known torsion (both signs, and the 0/pi
ends), and the features' chi mask and one-hot against a plain loop."""
import math

import numpy as np
import torch

from bindcraft2_amd import params as bparams
from oracle import af2

D = torch.float64


def _quad(theta):
    """b-c along x; a in the xy-plane; d rotated by theta about the b-c axis."""
    b = np.array([0.0, 0.0, 0.0])
    c = np.array([1.5, 0.0, 0.0])
    a = np.array([-0.5, 1.2, 0.0])
    d = c + np.array([0.6, 1.1 * math.cos(theta), 1.1 * math.sin(theta)])
    return [torch.tensor(v, dtype=D) for v in (a, b, c, d)]


def test_dihedral_known_torsions():
    for theta in (0.0, 0.3, 1.2, -0.7, -2.5, math.pi - 1e-9):
        got = float(af2.dihedral_angle(*_quad(theta)))
        # worked by hand for this construction: c1 = v1 x v2 = (0, 0, 1.8),
        # c2 = v3 x v2 = (0, -1.65 sin t, 1.65 cos t), c3 . v2 = 4.455 sin t,
        # |v2| (c1 . c2) = 4.455 cos t: the dihedral is +t
        want = math.atan2(math.sin(theta), math.cos(theta))
        assert abs(math.remainder(got - want, 2 * math.pi)) < 1e-9, theta


def test_template_row_mask_and_onehot_loop():
    rng = np.random.default_rng(0)
    tables = bparams.init_residue_tables(rng)
    prm = bparams.init_embedder_params(rng)
    n = 7
    aat = np.array([0, 5, 21, 20, 13, 7, 2])
    pos = 3 * rng.standard_normal((n, 37, 3))
    msk = (rng.random((n, 37)) < 0.85).astype(float)
    row, rmask = af2.template_row(aat, pos, msk, prm, tables)
    assert row.shape == (n, 256)
    for i in range(n):
        g = min(aat[i], 20)
        for c in range(4):
            idx = tables["chi_atom_indices"][g, c].astype(int)
            m = tables["chi_angles_mask"][g, c] * np.prod(msk[i, idx])
            if c == 0:
                assert float(rmask[i]) == m
    # one-hot of 22: the gap (21) has its own column
    P = af2.Params(prm, "param/", D)
    feat0 = torch.zeros(22, dtype=D)
    feat0[21] = 1.0
    h = torch.relu(feat0 @ P("template_single_embedding/weights")[:22] +
                   P("template_single_embedding/bias"))
    want = h @ P("template_projection/weights") + P("template_projection/bias")
    if float(rmask[2]) == 0.0:  # gap residue: no chi features
        np.testing.assert_allclose(row[2].numpy(), want.numpy(), rtol=1e-10)
