"""GPU parity of the design step's recycle terms (bc2n_probe_recycle,
modules_multimer.py:487-507) against the oracle's recycle_terms on the same
previous state.  Positions lie on a 1/8 A grid, so squared distances and
the squared breaks (3.25 + 1.25 b)^2 are exact in f32 and f64 alike and
both sides put every pair in the same distogram bin -- including pairs
exactly on a break, which lie in no bin.  Bars: f32 LayerNorm arithmetic,
max error 1e-4 relative to the term's scale."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2
from tests.helpers import weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64


@pytest.mark.parametrize("n,first", [(32, True), (32, False), (96, False)])
def test_recycle_terms_parity(cuda, n, first):
    print(f"recycle terms n={n} first={first}", flush=True)
    rng = np.random.default_rng(7700 + n + int(first))
    prm = bparams.init_embedder_params(rng)
    wdir = weights_dir(prm, f"rec_{n}_{int(first)}")
    pair0 = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa0 = rng.standard_normal((n, 256)).astype(np.float32)
    aat = rng.integers(0, 21, n).astype(np.float32)
    aat[::5] = 7  # glycines read CA
    atoms = (np.round(8 * 6.0 * rng.standard_normal((n, 14, 3))) / 8).astype(np.float32)
    atoms[3, 4] = atoms[0, 4] + np.array([4.5, 0, 0], np.float32)  # exactly on a break
    aat[0] = aat[3] = 0
    prev_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    prev_msa0 = rng.standard_normal((n, 256)).astype(np.float32)

    if first:
        z = (np.zeros((n, 14, 3)), np.zeros((n, n, 128)), np.zeros((n, 256)))
        pt, mt = af2.recycle_terms(np.zeros(n), *(torch.tensor(v, dtype=D) for v in z), prm)
    else:
        pt, mt = af2.recycle_terms(aat, torch.tensor(atoms, dtype=D),
                                   torch.tensor(prev_pair, dtype=D),
                                   torch.tensor(prev_msa0, dtype=D), prm)
    T = lambda a: torch.as_tensor(a, device=cuda)
    gp, gm = T(pair0.copy()), T(msa0.copy())
    if first:
        ops.probe_recycle(wdir, gp, gm)
    else:
        ops.probe_recycle(wdir, gp, gm, T(aat), T(atoms), T(prev_pair), T(prev_msa0))
    torch.cuda.synchronize()
    for name, g, base, t in (("pair", gp, pair0, pt), ("msa0", gm, msa0, mt)):
        got = g.cpu().double().numpy() - base
        want = t.numpy()
        err = np.abs(got - want).max() / np.abs(want).max()
        print(f"  {name} max rel err {err:.2e}")
        assert err <= 1e-4, name
    if not first:
        # the bins themselves: one distogram row per pair, the same on both sides
        dg = af2.dgram_from_positions(af2.pseudo_beta_atom14(aat, torch.tensor(atoms, dtype=D)))
        assert dg[0, 3].sum() == 0  # the pair exactly on a break
        assert dg.sum() > 0.2 * n * n  # most pairs lie in some bin
