"""GPU parity of the extra-MSA stack in its pair-only form (the reference's
native pair-only stack, bindcraft/af/native.py:1131-1193, used by the design
step where extra_msa_mask == 0).

The oracle runs the FULL extra-MSA EvoformerIteration
(modules_multimer.py:549-600 with is_extra_msa=True: c_e = 64, MSA row
attention with pair bias, global column attention, MSA transition, outer
product mean) on an all-zero extra-MSA mask, with every extra-MSA parameter
present; the GPU stack runs only the pair track plus the outer product mean's
constant output_b / 1e-3.  Agreement of the pair output and of d(pair)
therefore checks that reduction as well as the kernels."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64
C_E = 64


def _extra_params(depth, rng):
    prm = {}
    for b in range(depth):
        sh = bparams.module_shapes(c_m=C_E)
        sh.pop("msa_column_attention")
        sh["msa_column_global_attention"] = bparams.global_attention_shapes(C_E)
        for mod, shapes in sh.items():
            for pname, arr in bparams.init_module(shapes, rng, gates="random", ln="random").items():
                prm[f"param/block{b}/{mod}/{pname}"] = arr
        # with the mask at zero the outer product mean adds output_b / 1e-3 to
        # every pair entry; keep that constant O(0.1) so the pair modules see
        # the random pair rather than a per-channel offset pattern
        ob = f"param/block{b}/outer_product_mean/output_b"
        prm[ob] = (1e-4 * rng.standard_normal(prm[ob].shape)).astype(np.float32)
    return prm


def _opm_const(prm, depth):
    return sum(prm[f"param/block{b}/outer_product_mean/output_b"].astype(np.float64)
               for b in range(depth)) / 1e-3


@pytest.mark.parametrize("depth,n,s,dropout", [(1, 32, 1, False), (2, 64, 1, True),
                                               (2, 32, 3, True)])
def test_extra_stack_pair_only_parity(cuda, depth, n, s, dropout):
    print(f"extra stack depth={depth} n={n} s={s} dropout={dropout}", flush=True)
    rng = np.random.default_rng(4000 + depth * 100 + n + s)
    prm = _extra_params(depth, rng)
    wdir = weights_dir(prm, f"extra_{depth}_{n}_{s}")
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    emsa = rng.standard_normal((s, n, C_E)).astype(np.float32)
    pmask, _ = random_mask(n, 0.1, rng)
    emask = np.zeros((s, n), np.float32)  # the design step's extra MSA mask
    ct_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    key = J.prng_key(901 + n + s)

    st = ops.EvoformerStack(wdir, depth, pair_only=True, c_m=C_E)
    T = lambda a: torch.as_tensor(a, device=cuda)
    seed = ops.seed_tensor(key, enabled=True, device=cuda)
    po, _, save = st.forward(T(pair), T(emsa), T(pmask), T(emask), seed, dropout=dropout)
    dp, _ = st.backward(T(ct_pair), torch.zeros(s, n, C_E, device=cuda), T(pmask), T(emask), save,
                        seed, dropout=dropout)
    torch.cuda.synchronize()

    x = torch.tensor(pair, dtype=D, requires_grad=True)
    y = torch.tensor(emsa, dtype=D)
    _, rp = af2.evoformer_stack(y, x, torch.as_tensor(emask, dtype=D),
                                torch.as_tensor(pmask, dtype=D), prm, depth,
                                key if dropout else None, dropout, is_extra_msa=True)
    (gx,) = torch.autograd.grad(rp, x, torch.as_tensor(ct_pair, dtype=D))
    # compare the pair modules' updates: the outer product mean's constant
    # (identical on both sides) is taken out of both deltas
    c = torch.as_tensor(_opm_const(prm, depth))
    ref = rp.detach() - x.detach() - c
    print(" pair delta", assert_act(po.cpu().double() - x.detach() - c, ref, what="pair"),
          "|ref|/|pair|", (ref.norm() / x.detach().norm()).item())
    print(" dpair", assert_grad(dp.cpu().double(), gx, what="dpair"))
