"""Pins of the oracle's recycle terms (modules_multimer.py:487-507,
modules.py:1215-1264): the distogram against a plain loop over the squared
breaks, its edge cases (zero distance and a distance exactly on a break lie
in no bin), pseudo-beta's glycine rule, and the first pass's closed form (a
zero state gives the Linear's bias plus the pair norm's offset, and the msa
norm's offset)."""
import numpy as np
import torch

from bindcraft2_amd import params as bparams
from oracle import af2

D = torch.float64


def _loop_dgram(pos):
    n = pos.shape[0]
    lower = [(3.25 + 1.25 * b) ** 2 for b in range(15)]
    upper = lower[1:] + [1e8]
    out = np.zeros((n, n, 15))
    for i in range(n):
        for j in range(n):
            d2 = sum((pos[i][c] - pos[j][c]) ** 2 for c in range(3))
            for b in range(15):
                if lower[b] < d2 < upper[b]:
                    out[i, j, b] = 1.0
    return out


def test_dgram_matches_loop_and_edges():
    rng = np.random.default_rng(0)
    pos = 12.0 * rng.standard_normal((9, 3))
    got = af2.dgram_from_positions(torch.tensor(pos, dtype=D)).numpy()
    np.testing.assert_array_equal(got, _loop_dgram(pos))
    assert got.sum(-1).max() <= 1.0
    # zero distance: no bin (the diagonal); a distance on a break: no bin
    assert got[np.arange(9), np.arange(9)].sum() == 0
    on = np.array([[0.0, 0.0, 0.0], [4.5, 0.0, 0.0], [0.0, 30.0, 0.0]])
    g = af2.dgram_from_positions(torch.tensor(on, dtype=D)).numpy()
    assert g[0, 1].sum() == 0          # exactly the second break
    assert g[0, 2, 14] == 1.0          # past the last break: the open bin


def test_pseudo_beta_glycine_rule():
    rng = np.random.default_rng(1)
    a14 = torch.tensor(rng.standard_normal((4, 14, 3)), dtype=D)
    aat = np.array([7, 0, 7, 19])
    pb = af2.pseudo_beta_atom14(aat, a14)
    assert torch.equal(pb[0], a14[0, 1]) and torch.equal(pb[2], a14[2, 1])
    assert torch.equal(pb[1], a14[1, 4]) and torch.equal(pb[3], a14[3, 4])


def test_first_pass_terms_closed_form():
    rng = np.random.default_rng(2)
    prm = bparams.init_embedder_params(rng)
    n = 5
    pair_t, msa_t = af2.recycle_terms(np.zeros(n), torch.zeros(n, 14, 3, dtype=D),
                                      torch.zeros(n, n, 128, dtype=D),
                                      torch.zeros(n, 256, dtype=D), prm)
    want_pair = prm["param/prev_pos_linear/bias"] + prm["param/prev_pair_norm/offset"]
    np.testing.assert_allclose(pair_t.numpy(), np.broadcast_to(want_pair, (n, n, 128)), rtol=1e-6)
    np.testing.assert_allclose(msa_t.numpy(),
                               np.broadcast_to(prm["param/prev_msa_first_row_norm/offset"],
                                               (n, 256)), rtol=1e-6)


def test_recycle_terms_pick_one_weight_row():
    """With the norms' inputs zero, the pair term is bias + offset + the
    prev_pos_linear row of the pair's bin."""
    rng = np.random.default_rng(3)
    prm = bparams.init_embedder_params(rng)
    a14 = torch.zeros(2, 14, 3, dtype=D)
    a14[1, 4, 0] = 6.0   # CB of residue 1 at 6 A: bin 2 (5.75 < 6 < 7)
    pair_t, _ = af2.recycle_terms(np.array([0, 0]), a14, torch.zeros(2, 2, 128, dtype=D),
                                  torch.zeros(2, 256, dtype=D), prm)
    base = prm["param/prev_pos_linear/bias"] + prm["param/prev_pair_norm/offset"]
    np.testing.assert_allclose(pair_t[0, 1].numpy(), base + prm["param/prev_pos_linear/weights"][2],
                               rtol=1e-6)
    np.testing.assert_allclose(pair_t[0, 0].numpy(), base, rtol=1e-6)
