"""Pins of the oracle's confidence metrics (oracle/af2.py confidence,
_tm_score) by closed forms and brute force: bin-delta logits give the bin
centres and the TM-score of a known distance; a single chain has ipTM 0;
pTM against a pure-Python loop over the TM-score definition; pLDDT of
uniform logits is 0.5; PAE is symmetric; finite differences of every
output."""
import math

import numpy as np
import torch

from oracle import af2

D = torch.float64


def _delta(n, bins, at):
    x = torch.full((n, n, bins), -30.0, dtype=D)
    x[..., at] = 30.0
    return x


def test_delta_bins_give_centres_and_tm():
    n = 24
    lg = _delta(n, 64, 10)
    out = af2.confidence(torch.zeros(n, 50, dtype=D), lg, torch.zeros(n, 37, dtype=D),
                         torch.ones(n, dtype=D), np.zeros(n, np.int32))
    plddt, pae, ptm, iptm, iptm_pr, ex = out
    np.testing.assert_allclose(plddt.numpy(), 0.5, atol=1e-12)
    np.testing.assert_allclose(pae.numpy(), 0.5 * 10 + 0.25, atol=1e-9)
    d0 = 1.24 * (24 - 15) ** (1 / 3) - 1.8
    np.testing.assert_allclose(ptm.item(), 1 / (1 + 5.25 ** 2 / d0 ** 2), rtol=1e-9)
    assert iptm.item() == 0.0 and float(iptm_pr.abs().max()) == 0.0  # one chain
    np.testing.assert_allclose(ex.numpy(), 0.5)


def test_tm_score_brute_force():
    rng = np.random.default_rng(0)
    n = 7
    lg = rng.standard_normal((n, n, 64))
    w = rng.uniform(0.2, 1.0, n)
    asym = np.array([0, 0, 0, 1, 1, 2, 2])
    breaks = np.linspace(0, 31, 63)
    centres = list(breaks + 0.25) + [31.75]
    d0 = 1.24 * (max(w.sum(), 19) - 15) ** (1 / 3) - 1.8
    for use_asym in (False, True):
        per = []
        for i in range(n):
            num = den = 0.0
            for j in range(n):
                m = 1.0 if not use_asym else float(asym[i] != asym[j])
                p = np.exp(lg[i, j] - lg[i, j].max())
                p /= p.sum()
                t = sum(p[b] / (1 + centres[b] ** 2 / d0 ** 2) for b in range(64))
                num += t * m * m * w[i] * w[j]
                den += m * w[i] * w[j]
            per.append(num / (1e-8 + den))
        want = max(per[i] * w[i] for i in range(n))
        got, got_per = af2._tm_score(torch.tensor(lg, dtype=D), torch.tensor(breaks, dtype=D),
                                     torch.tensor(w, dtype=D), asym if use_asym else None)
        np.testing.assert_allclose(got.item(), want, rtol=1e-12)
        np.testing.assert_allclose(got_per.numpy(), per, rtol=1e-12)


def test_symmetric_pae_and_gradients():
    rng = np.random.default_rng(1)
    n = 5
    args = [torch.tensor(rng.standard_normal(s), dtype=D, requires_grad=True)
            for s in ((n, 50), (n, n, 64), (n, 37))]
    mask = torch.tensor([1, 1, 0.5, 1, 1], dtype=D)
    asym = np.array([0, 0, 1, 1, 1], np.int32)
    out = af2.confidence(*args, mask, asym)
    np.testing.assert_allclose(out[1].detach().numpy(), out[1].detach().numpy().T)
    fn = lambda a, b, c: sum(o.sum() * (k + 1) for k, o in enumerate(af2.confidence(a, b, c, mask, asym)))
    assert torch.autograd.gradcheck(fn, tuple(args), eps=1e-6, atol=1e-7)
