"""GPU parity of bc2n_confidence_* (pLDDT, PAE, pTM, ipTM and per residue,
CA experimentally-resolved) against the oracle's confidence
(bindcraft/af2.py:197-219 with AF2's predicted_tm_score), forward and the
backward of every output, f32 against fp64 within 1e-5 relative; N = 37
leaves a partial group of pairs, N = 64 fills them; masked residues and
three chains exercise the masks."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops
from oracle import af2

pytestmark = pytest.mark.gpu
D = torch.float64


@pytest.mark.parametrize("n", [37, 64])
def test_confidence_parity(cuda, n):
    print(f"confidence n={n}", flush=True)
    rng = np.random.default_rng(n)
    lg = [(2 * rng.standard_normal(s)).astype(np.float32) for s in ((n, 50), (n, n, 64), (n, 37))]
    mask = np.ones(n, np.float32)
    mask[rng.choice(n, 3, replace=False)] = 0.0
    asym = np.repeat([0, 1, 2], [n // 3, n // 3, n - 2 * (n // 3)]).astype(np.int32)
    cts = [rng.standard_normal(s).astype(np.float32) for s in ((n,), (n, n), (1,), (1,), (n,), (n,))]
    T = lambda a: torch.as_tensor(a, device=cuda)
    op = ops.Confidence()
    outs, save = op.forward(*map(T, lg), T(mask), T(asym))
    d = op.backward([T(c) for c in cts], *map(T, lg), T(mask), T(asym), save)
    torch.cuda.synchronize()

    ts = [torch.tensor(x, dtype=D, requires_grad=True) for x in lg]
    ref = af2.confidence(*ts, torch.tensor(mask, dtype=D), asym)
    loss = sum((r * torch.tensor(c, dtype=D)).sum() for r, c in zip(ref, cts))
    grads = torch.autograd.grad(loss, ts)
    names = ("plddt", "pae", "ptm", "iptm", "iptm_per_residue", "expres_ca",
             "d plddt_logits", "d pae_logits", "d expres_logits")
    for name, g, r in zip(names, list(outs) + list(d), [x.detach() for x in ref] + list(grads)):
        g = g.cpu().double()
        err = ((g - r).norm() / r.norm().clamp_min(1e-30)).item()
        print(f"  {name}: rel {err:.2e}")
        assert err <= 1e-5, name
