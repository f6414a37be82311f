"""GPU parity of the structure module + heads (the drop-in for
StructureHeadsFwd/Bwd, native/ffi.cu:1009-1044) through the C ABI against the
fp64 oracle: fold iterations (folding_multimer.py:476-548), the last
iteration's sidechain (:950-1040 with all_atom_multimer.py:370-468) and the
four heads (modules.py:777-1120).

f32 end to end, so the bar is the fold's: outputs relL2 <= 1e-3 (random
weights amplify rounding through the frame composition), gradients cosine
>= 0.9999.  The residue tables are random rigid frames and positions: the
sidechain is table-driven, and the oracle's frame algebra is pinned against
4x4 homogeneous products (tests/test_oracle_af2.py)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64
NAMES = ("atom14", "distogram", "pae", "plddt", "expres")


def _case(n, seed, mask_frac):
    rng = np.random.default_rng(seed)
    prm = bparams.init_structure_heads_params(rng, final="random", ln="random")
    tables = bparams.init_residue_tables(rng)
    for k, v in tables.items():
        prm[f"const/{k}"] = v
    wdir = weights_dir(prm, f"sh_{n}_{seed}")
    single = rng.standard_normal((n, 384)).astype(np.float32)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    mask = np.ones(n, np.float32)
    k = int(round(mask_frac * n))
    if k:
        mask[rng.choice(n, k, replace=False)] = 0.0
    aatype = rng.integers(0, 21, n).astype(np.float32)
    return rng, prm, tables, wdir, single, pair, mask, aatype


@pytest.mark.parametrize("n,depth,dropout,mask_frac", [
    (32, 1, False, 0.0), (48, 2, True, 0.1), (64, 3, True, 0.0),
    # the longest length the entry point takes
    (1024, 2, True, 0.1),
])
def test_structure_heads_fwd_bwd_parity(cuda, n, depth, dropout, mask_frac):
    print(f"structure heads n={n} depth={depth} dropout={dropout} mask={mask_frac}", flush=True)
    rng, prm, tables, wdir, single, pair, mask, aatype = _case(n, 50 + n + depth, mask_frac)
    key = J.prng_key(2000 + n)
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))
    cts = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    mod = ops.StructureHeads(wdir, depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    seed = ops.seed_tensor(key, dropout, cuda)
    outs, save = mod.forward(T(single), T(pair), T(mask), T(aatype), seed, dropout=dropout)
    ds, dz = mod.backward([T(c) for c in cts], T(single), T(pair), T(mask), T(aatype), save,
                          dropout=dropout)
    torch.cuda.synchronize()

    s = torch.tensor(single, dtype=D, requires_grad=True)
    z = torch.tensor(pair, dtype=D, requires_grad=True)
    ref = af2.structure_heads(s, z, torch.as_tensor(mask, dtype=D), aatype, prm, depth, key,
                              dropout, tables)
    loss = sum((r * torch.as_tensor(c, dtype=D)).sum() for r, c in zip(ref, cts))
    gs, gz = torch.autograd.grad(loss, (s, z))
    for name, o, r in zip(NAMES, outs, ref):
        print(" ", name, assert_act(o.cpu().double(), r.detach(), 1e-3, name))
    print("  dsingle", assert_grad(ds.cpu().double(), gs, 0.9999, "dsingle"))
    print("  dpair", assert_grad(dz.cpu().double(), gz, 0.9999, "dpair"))


def test_structure_heads_null_cotangents(cuda):
    """Absent cotangents count as zero: the atom14 cotangent alone, then the
    heads' alone, each against the oracle with the others zeroed."""
    n, depth = 32, 2
    rng, prm, tables, wdir, single, pair, mask, aatype = _case(n, 77, 0.0)
    mod = ops.StructureHeads(wdir, depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    outs, save = mod.forward(T(single), T(pair), T(mask), T(aatype), None, dropout=False)
    s = torch.tensor(single, dtype=D, requires_grad=True)
    z = torch.tensor(pair, dtype=D, requires_grad=True)
    ref = af2.structure_heads(s, z, torch.as_tensor(mask, dtype=D), aatype, prm, depth, None,
                              False, tables)
    for keep in ((0,), (1, 2, 3, 4)):
        cts = [rng.standard_normal(tuple(o.shape)).astype(np.float32) if i in keep else None
               for i, o in enumerate(outs)]
        ds, dz = mod.backward([None if c is None else T(c) for c in cts], T(single), T(pair),
                              T(mask), T(aatype), save, dropout=False)
        torch.cuda.synchronize()
        loss = sum((r * torch.as_tensor(c, dtype=D)).sum() for r, c in zip(ref, cts) if c is not None)
        gs, gz = torch.autograd.grad(loss, (s, z), retain_graph=True)
        print(" keep", keep, assert_grad(ds.cpu().double(), gs, 0.9999, "dsingle"),
              assert_grad(dz.cpu().double(), gz, 0.9999, "dpair"))
