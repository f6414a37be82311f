"""GPU parity of the structure module's fold iterations (IPA + transition +
quaternion rigid update, folding_multimer.py:188-548) through the C ABI
against the fp64 oracle on the same seeded inputs, weights and JAX dropout
keys.  The path is f32 end to end (as AF2 runs it), so the bars are f32-level,
tighter than the trunk's bf16 ones."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import metrics, weights_dir

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,batch,ta,tb", [
    (64, 64, 16, 1, False, False), (37, 53, 29, 1, True, False), (100, 40, 300, 3, False, True),
    (512, 12, 128, 1, False, False), (70, 33, 70, 12, True, True),
])
def test_gemm_f32(cuda, M, N, K, batch, ta, tb):
    """Batched strided f32 MFMA GEMM against torch fp64 matmul."""
    print(f"gemm_f32 M={M} N={N} K={K} batch={batch} ta={ta} tb={tb}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N)
    A = torch.randn(batch, K, M, generator=g) if ta else torch.randn(batch, M, K, generator=g)
    B = torch.randn(batch, N, K, generator=g) if tb else torch.randn(batch, K, N, generator=g)
    ref = torch.matmul(A.transpose(1, 2).double() if ta else A.double(),
                       B.transpose(1, 2).double() if tb else B.double())
    a_str = (1, M, M * K) if ta else (K, 1, M * K)
    b_str = (1, K, N * K) if tb else (N, 1, N * K)
    C = torch.empty(batch, M, N, device=cuda)
    ops.probe_gemm_f32(A.to(cuda), B.to(cuda), C, M, N, K, batch, a_str, b_str, (N, 1, M * N))
    m = metrics(C.cpu().double(), ref)
    assert m["rel_l2"] < 1e-5, m


def _case(n, seed, mask_frac):
    rng = np.random.default_rng(seed)
    prm = bparams.init_fold_params(rng, final="random", ln="random")
    wdir = weights_dir(prm, f"fold_{n}_{seed}")
    single = rng.standard_normal((n, 384)).astype(np.float32)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    mask = np.ones(n, np.float32)
    k = int(round(mask_frac * n))
    if k:
        mask[rng.choice(n, k, replace=False)] = 0.0
    d_act = rng.standard_normal((n, 384)).astype(np.float32)
    return prm, wdir, single, pair, mask, d_act, rng


def _oracle(prm, single, pair, mask, depth, key, dropout, d_act, d_traj):
    s = torch.tensor(single, dtype=torch.float64, requires_grad=True)
    z = torch.tensor(pair, dtype=torch.float64, requires_grad=True)
    m = torch.as_tensor(mask, dtype=torch.float64)
    act, traj = af2.fold(s, z, m, prm, depth, key, dropout)
    loss = (act * torch.as_tensor(d_act, dtype=torch.float64)).sum() + \
        (traj * torch.as_tensor(d_traj, dtype=torch.float64)).sum()
    ds, dz = torch.autograd.grad(loss, (s, z))
    return act.detach(), traj.detach(), ds, dz


@pytest.mark.parametrize("n,depth,dropout,mask_frac", [
    (32, 1, False, 0.0), (32, 2, True, 0.1), (64, 3, True, 0.2), (96, 2, False, 0.1),
    # the 8-layer structure module on an L=512 pair
    (512, 8, True, 0.1), (768, 2, True, 0.1), (1024, 2, True, 0.1),
])
def test_fold_fwd_bwd_parity(cuda, n, depth, dropout, mask_frac):
    print(f"fold n={n} depth={depth} dropout={dropout} mask={mask_frac}", flush=True)
    prm, wdir, single, pair, mask, d_act, rng = _case(n, 11 + n + depth, mask_frac)
    d_traj = (0.1 * rng.standard_normal((depth, n, 3, 4))).astype(np.float32)
    key = J.prng_key(1000 + n)
    mod = ops.Fold(wdir, depth)
    ts = torch.as_tensor(single, device=cuda)
    tz = torch.as_tensor(pair, device=cuda)
    tm = torch.as_tensor(mask, device=cuda)
    seed = ops.seed_tensor(key, dropout, cuda)
    act, traj, save = mod.forward(ts, tz, tm, seed, dropout=dropout)
    ds, dz = mod.backward(torch.as_tensor(d_act, device=cuda), torch.as_tensor(d_traj, device=cuda),
                          ts, tz, tm, save, dropout=dropout)
    torch.cuda.synchronize()
    r_act, r_traj, r_ds, r_dz = _oracle(prm, single, pair, mask, depth, key if dropout else None,
                                        dropout, d_act, d_traj)
    ma, mt = metrics(act.cpu(), r_act), metrics(traj.cpu(), r_traj)
    ms, mz = metrics(ds.cpu(), r_ds), metrics(dz.cpu(), r_dz)
    print("  act", ma, "\n  traj", mt, "\n  dsingle", ms, "\n  dpair", mz)
    assert ma["rel_l2"] < 1e-3 and ma["max_rel"] < 1e-2, ma
    assert mt["rel_l2"] < 1e-3 and mt["max_rel"] < 1e-2, mt
    assert ms["cos"] > 0.9999 and ms["rel_l2"] < 1e-2, ms
    assert mz["cos"] > 0.9999 and mz["rel_l2"] < 1e-2, mz


def test_fold_zero_cotangents(cuda):
    """d_act = d_traj = None gives exactly zero gradients."""
    prm, wdir, single, pair, mask, _, _ = _case(32, 5, 0.0)
    mod = ops.Fold(wdir, 2)
    ts, tz, tm = (torch.as_tensor(x, device=cuda) for x in (single, pair, mask))
    _, _, save = mod.forward(ts, tz, tm, None, dropout=False)
    ds, dz = mod.backward(None, None, ts, tz, tm, save, dropout=False)
    assert torch.count_nonzero(ds).item() == 0 and torch.count_nonzero(dz).item() == 0
