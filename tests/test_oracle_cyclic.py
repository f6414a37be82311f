"""Pins of the oracle's cyclic sequence offsets and target flexibility
(bindcraft/af2.py:150-185), CPU only.

The offsets are checked against a brute-force choice on the ring (of the
displacements d, d - L, d + L the shortest, a tie keeping d), not against
the min/where formula they restate; flexibility f = 1/k against its closed
form (every k-th residue index, counting from 1)."""
import numpy as np
import torch

from bindcraft2_amd import params as bparams
from oracle import af2


def _ring(d, L, mode):
    cands = sorted((d, d - L, d + L), key=lambda v: (abs(v), v != d))
    best = cands[0]
    if mode == "distance":
        return int(np.sign(d)) * abs(best)
    if mode == "neighbours" and abs(best) > 2:
        return 32 * int(np.sign(best))
    return best


def test_cyclic_offsets_against_ring_brute_force():
    # chain 1: 9 cyclic residues (one masked), chain 2: 6 plain, chain 3: 8 cyclic (even ring)
    ri = np.concatenate([np.arange(9), np.arange(6), np.arange(8)])
    asym = np.repeat([1, 2, 3], [9, 6, 8])
    flags = np.zeros(23, np.int64)
    flags[asym == 1] |= af2.CYCLIC
    flags[asym == 3] |= af2.CYCLIC
    mask = np.ones(23)
    mask[4] = 0.0  # a masked residue leaves the ring (and shortens it)
    for mode in af2.CYCLIC_MODES:
        got = af2.cyclic_sequence_offsets(ri, asym, flags, mask, mode)
        for i in range(23):
            for j in range(23):
                d = int(ri[i] - ri[j])
                cyclic = (asym[i] == asym[j] and asym[i] != 2 and mask[i] and mask[j])
                if not cyclic:
                    want = d
                else:
                    L = int(((asym == asym[i]) * mask).sum())
                    want = _ring(d, L, mode)
                assert got[i, j] == want, (mode, i, j, got[i, j], want)


def test_flexibility_selects_every_kth_template_residue():
    ri = np.arange(40)
    tmask = np.ones(40, bool)
    tmask[:10] = False  # not template (or designed)
    for k in (2, 3, 4, 7):
        got = af2.flexible_target_residues(ri, tmask, 1.0 / k)
        want = tmask & ((ri + 1) % k == 0)
        np.testing.assert_array_equal(got, want)
    assert not af2.flexible_target_residues(ri, tmask, 0.0).any()


def test_flexible_residue_is_a_template_gap():
    """A flexible template residue's MSA row is the row of a gap: one-hot 21
    and no chi features, whatever its atoms."""
    rng = np.random.default_rng(3)
    tables = bparams.init_residue_tables(rng)
    prm = bparams.init_embedder_params(rng)
    n = 6
    aat = np.array([3, 7, 21, 11, 0, 19])
    pos = 3 * rng.standard_normal((n, 37, 3))
    msk = np.ones((n, 37))
    row, rmask = af2.template_row(aat, pos, msk, prm, tables)
    assert rmask[2] == 0
    # residue 4 made a gap as flexibility does: aatype 21, side chain unmasked out
    aat2 = aat.copy()
    aat2[4] = 21
    msk2 = msk.copy()
    msk2[4, 5:] = 0
    row2, _ = af2.template_row(aat2, pos, msk2, prm, tables)
    torch.testing.assert_close(row2[4], row[2], rtol=0, atol=1e-12)


def test_frames_from_atoms_recovers_the_rotation():
    """A backbone triple in the canonical frame (C on +x, N in the xy plane
    with y > 0, CA at 0) moved by a rotation Q and a shift s gives back
    R = Q and t = s / position_scale; an all-zero residue (no atoms) gives
    the zero matrix, as the multimer model's Gram-Schmidt does."""
    from scipy.spatial.transform import Rotation
    rng = np.random.default_rng(5)
    can = np.array([[-0.52, 1.36, 0.0], [0.0, 0.0, 0.0], [1.52, 0.0, 0.0]])  # N, CA, C
    Q = Rotation.random(4, random_state=7).as_matrix()
    s = 10 * rng.standard_normal((4, 3))
    pos = np.zeros((5, 37, 3))
    for i in range(4):
        pos[i, :3] = can @ Q[i].T + s[i]
    R, t = af2.frames_from_atoms(torch.as_tensor(pos))
    torch.testing.assert_close(R[:4], torch.as_tensor(Q), rtol=0, atol=1e-12)
    torch.testing.assert_close(t[:4], torch.as_tensor(s) / af2.POSITION_SCALE, rtol=0, atol=1e-12)
    assert torch.equal(R[4], torch.zeros(3, 3, dtype=R.dtype)) and not t[4].any()
