"""Pins of the oracle's alignment of the design step's atoms
(bindcraft/protein.py:75-83 kabsch, bindcraft/af2.py:89-97) and its atom37
gather: scipy's weighted Rotation.align_vectors (an independent solver), an
exact rigid motion recovered exactly, a mirror image still aligned by a
proper rotation, no weights giving the identity, and the gather against a
plain loop."""
import numpy as np
import torch
from scipy.spatial.transform import Rotation

from bindcraft2_amd import params as bparams
from oracle import af2

D = torch.float64


def _rot(rng):
    return Rotation.random(random_state=int(rng.integers(1 << 30))).as_matrix()


def test_kabsch_matches_scipy_weighted():
    rng = np.random.default_rng(0)
    x = 5 * rng.standard_normal((20, 3))
    y = x @ _rot(rng).T + rng.standard_normal(3) + 0.3 * rng.standard_normal((20, 3))
    w = (rng.random(20) < 0.7).astype(float)
    R, xc, yc = af2.kabsch(torch.tensor(x, dtype=D), torch.tensor(y, dtype=D), torch.tensor(w))
    xm = (x * w[:, None]).sum(0) / w.sum()
    ym = (y * w[:, None]).sum(0) / w.sum()
    rs, _ = Rotation.align_vectors(y - ym, x - xm, weights=w)
    np.testing.assert_allclose(R.numpy(), rs.as_matrix(), atol=1e-9)
    np.testing.assert_allclose(xc.numpy(), xm, rtol=1e-7)
    assert abs(np.linalg.det(R.numpy()) - 1) < 1e-12


def test_kabsch_rigid_motion_and_mirror_and_empty():
    rng = np.random.default_rng(1)
    x = 4 * rng.standard_normal((12, 3))
    R0, t0 = _rot(rng), rng.standard_normal(3)
    y = x @ R0.T + t0
    w = torch.ones(12)
    R, xc, yc = af2.kabsch(torch.tensor(x, dtype=D), torch.tensor(y, dtype=D), w)
    np.testing.assert_allclose(((torch.tensor(x) - xc) @ R.T + yc).numpy(), y, atol=1e-9)
    # a mirror image: the best proper rotation, never the reflection
    Rm, _, _ = af2.kabsch(torch.tensor(x, dtype=D), torch.tensor(-y, dtype=D), w)
    assert abs(np.linalg.det(Rm.numpy()) - 1) < 1e-12
    # no weight at all: the identity, and the centres are zero
    Re, xe, ye = af2.kabsch(torch.tensor(x, dtype=D), torch.tensor(y, dtype=D), torch.zeros(12))
    np.testing.assert_allclose(Re.numpy(), np.eye(3), atol=1e-12)
    assert float(xe.abs().max()) == 0.0 and float(ye.abs().max()) == 0.0


def test_atom37_gather_loop():
    rng = np.random.default_rng(2)
    tables = bparams.init_residue_tables(rng)
    n = 6
    a14 = torch.tensor(rng.standard_normal((n, 14, 3)), dtype=D)
    aat = rng.integers(0, 21, n)
    sm = torch.tensor([1, 1, 0, 1, 1, 1], dtype=D)
    a37, ex = af2.atom14_to_atom37(a14, aat, sm, tables)
    for i in range(n):
        for a in range(37):
            e = tables["atom37_mask"][aat[i], a] * float(sm[i])
            assert float(ex[i, a]) == e
            want = a14[i, int(tables["atom37_to_atom14"][aat[i], a])] * e
            assert torch.equal(a37[i, a], want)
