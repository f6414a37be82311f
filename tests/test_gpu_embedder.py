"""GPU parity of the multimer input embedder (the drop-in for EmbedderFwd /
EmbedderBwd, native/ffi.cu:1046-1071) through the C ABI against the fp64
oracle (modules_multimer.py:358-483 with the native feature mask,
native/embed.cuh:187-195).

Everything on both sides is f32 / fp64 arithmetic with K <= 49 (no bf16), so
the bar is f32 round-off: relative L2 and normwise max error <= 1e-5 on msa,
pair, d(target_feat) and d(msa_feat)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2
from tests.helpers import assert_act, weights_dir

pytestmark = pytest.mark.gpu
F32_TOL = 1e-5


def _ids(n, chains, same_entity):
    """`chains` chains of near-equal length; residue_index restarts per chain
    (and jumps by 40 inside the first, to reach the clipped bins)."""
    cut = np.array_split(np.arange(n), chains)
    ri, ai, ei, si = (np.zeros(n, np.float32) for _ in range(4))
    for c, idx in enumerate(cut):
        r = np.arange(len(idx), dtype=np.float32)
        if c == 0:
            r[len(idx) // 2:] += 40
        ri[idx], ai[idx] = r, c + 1
        ei[idx] = 1 if same_entity else c + 1
        si[idx] = c + 1 if same_entity else 1
    return ri, ai, ei, si


@pytest.mark.parametrize("n,s,chains,same_entity,use_offset,pad", [
    (32, 1, 1, True, False, 0),
    (50, 3, 2, True, False, 2),
    (64, 2, 3, False, True, 1),
    (224, 1, 2, False, False, 0),
    (224, 5, 2, True, True, 3),
])
def test_embedder_fwd_bwd_parity(cuda, n, s, chains, same_entity, use_offset, pad):
    print(f"embedder n={n} s={s} chains={chains} same_entity={same_entity} "
          f"offset={use_offset} pad={pad}", flush=True)
    rng = np.random.default_rng(7000 + n + s)
    prm = bparams.init_embedder_params(rng, scoped=bool(n % 2))
    wdir = weights_dir(prm, f"emb_{n}_{s}_{chains}")
    tf = np.zeros((n, 21), np.float32)
    tf[:, :20] = rng.dirichlet(np.ones(20), n)
    if pad:
        tf[-pad:] = 0.0  # padded residues: their preprocess_1d rows are zeroed
    mf = rng.standard_normal((s, n, 49)).astype(np.float32)
    ri, ai, ei, si = _ids(n, chains, same_entity)
    off = rng.integers(-45, 46, (n, n)).astype(np.int32) if use_offset else None
    dmsa = rng.standard_normal((s, n, 256)).astype(np.float32)
    dpair = rng.standard_normal((n, n, 128)).astype(np.float32)

    T = lambda a: torch.as_tensor(a, device=cuda)
    emb = ops.Embedder(wdir)
    msa, pair = emb.forward(T(tf), T(mf), T(ri), T(ai), T(ei), T(si),
                            T(off) if off is not None else None)
    dtf, dmf = emb.backward(T(dmsa), T(dpair), T(tf))
    torch.cuda.synchronize()

    D = torch.float64
    tft = torch.tensor(tf, dtype=D, requires_grad=True)
    mft = torch.tensor(mf, dtype=D, requires_grad=True)
    rmsa, rpair = af2.embedder(tft, mft, ri, ai, ei, si, prm, offset=off)
    gtf, gmf = torch.autograd.grad((rmsa, rpair), (tft, mft),
                                   (torch.as_tensor(dmsa, dtype=D), torch.as_tensor(dpair, dtype=D)))
    print(" msa", assert_act(msa.cpu().double(), rmsa.detach(), F32_TOL, "msa"))
    print(" pair", assert_act(pair.cpu().double(), rpair.detach(), F32_TOL, "pair"))
    print(" dtf", assert_act(dtf.cpu().double(), gtf, F32_TOL, "dtarget_feat"))
    print(" dmf", assert_act(dmf.cpu().double(), gmf, F32_TOL, "dmsa_feat"))
    if pad:
        # the feature mask: padded rows' msa is exactly preprocess_msa's
        P = af2.Params(prm, "param/")
        pm = af2.linear(torch.as_tensor(mf, dtype=D), P.sub("preprocess_msa/"))
        assert_act(msa[:, -pad:].cpu().double(), pm[:, -pad:], F32_TOL, "masked msa rows")


def test_embedder_rejects_bad_operands(cuda):
    prm = bparams.init_embedder_params(np.random.default_rng(1))
    emb = ops.Embedder(weights_dir(prm, "emb_bad"))
    z = torch.zeros(8, 21, device=cuda)
    with pytest.raises(RuntimeError):
        emb.forward(z, torch.zeros(0, 8, 49, device=cuda), *(torch.zeros(8, device=cuda),) * 4)
