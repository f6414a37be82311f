"""The save-set survives an intervening forward (the reference's stack gate,
native/tplstack.cu:1-17; the reason the save-set crosses the FFI as a value,
native/ffi.cu:17-25): forward(A), then forward(B) on other data, then
backward(A) from A's save-set must give exactly the bits of a backward taken
right after forward(A).  JAX dispatches asynchronously, so a second forward
can overtake the first backward; state kept inside the library (scratch,
weights, keys) must not carry anything the backward reads.

Run for the Evoformer stack (main and pair-only), the template pair stack,
the template embedding and the one-call design step."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import jax_prng as J
from tests.helpers import random_mask, weights_dir
from tests.test_gpu_design_step import _extra_params

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"{what}: output {i} changed by the intervening forward"


@pytest.mark.parametrize("pair_only", [False, True])
def test_evoformer_save_survives(cuda, pair_only):
    n, s, depth = 64, 2, 2
    print(f"evoformer fwd(A) fwd(B) bwd(A) n={n} depth={depth} pair_only={pair_only}", flush=True)
    rng = np.random.default_rng(71 + pair_only)
    if pair_only:
        prm, cm = _extra_params(depth, rng), 64
    else:
        prm, cm = {}, 256
        for b in range(depth):
            prm.update(bparams.init_block_params(b, rng, gates="random", ln="random"))
    st = ops.EvoformerStack(weights_dir(prm, f"survive_evo{int(pair_only)}"), depth,
                            pair_only=pair_only, c_m=cm)
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask, m1 = random_mask(n, 0.1, rng)
    mmask = T(np.tile(m1, (s, 1)).astype(np.float32))
    pmask = T(pmask)

    def inputs():
        return (T(rng.standard_normal((n, n, 128)).astype(np.float32)),
                T(rng.standard_normal((s, n, cm)).astype(np.float32)))

    (pa, ma), (pb, mb) = inputs(), inputs()
    ct_p, ct_m = torch.randn_like(pa), torch.randn_like(ma)
    sa, sb = ops.seed_tensor(J.prng_key(5), True, cuda), ops.seed_tensor(J.prng_key(6), True, cuda)
    _, _, save = st.forward(pa, ma, pmask, mmask, sa)
    ref = [t.clone() for t in st.backward(ct_p, ct_m, pmask, mmask, save, sa)]
    _, _, save_a = st.forward(pa, ma, pmask, mmask, sa)
    _, _, save_b = st.forward(pb, mb, pmask, mmask, sb)
    got = st.backward(ct_p, ct_m, pmask, mmask, save_a, sa)
    torch.cuda.synchronize()
    _same(ref, got, "evoformer")
    assert not torch.equal(save_a, save_b)


def test_template_stack_save_survives(cuda):
    n, depth = 64, 2
    print(f"template stack fwd(A) fwd(B) bwd(A) n={n} depth={depth}", flush=True)
    rng = np.random.default_rng(73)
    prm = {}
    for b in range(depth):
        prm.update(bparams.init_template_block_params(b, rng, gates="random", ln="random"))
    st = ops.TemplatePairStack(weights_dir(prm, "survive_tpl"), depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask = T(random_mask(n, 0.1, rng)[0])
    xa = T(rng.standard_normal((n, n, 64)).astype(np.float32))
    xb = T(rng.standard_normal((n, n, 64)).astype(np.float32))
    ct = torch.randn_like(xa)
    sa, sb = ops.seed_tensor(J.prng_key(7), True, cuda), ops.seed_tensor(J.prng_key(8), True, cuda)
    _, save = st.forward(xa, pmask, sa)
    ref = st.backward(ct, pmask, save, sa).clone()
    _, save_a = st.forward(xa, pmask, sa)
    st.forward(xb, pmask, sb)
    got = st.backward(ct, pmask, save_a, sa)
    torch.cuda.synchronize()
    _same([ref], [got], "template stack")


def test_template_embedding_save_survives(cuda):
    n, depth = 64, 2
    print(f"template embedding fwd(A) fwd(B) bwd(A) n={n} depth={depth}", flush=True)
    rng = np.random.default_rng(74)
    prm = bparams.init_template_embedding_params(depth, rng, gates="random", ln="random")
    te = ops.TemplateEmbedding(weights_dir(prm, "survive_tpe"), depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask = T(random_mask(n, 0.1, rng)[0])
    qa = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    qb = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    ca = T(rng.standard_normal((n, n, 64)).astype(np.float32))
    cb = T(rng.standard_normal((n, n, 64)).astype(np.float32))
    ct = torch.randn_like(qa)
    sa, sb = ops.seed_tensor(J.prng_key(9), True, cuda), ops.seed_tensor(J.prng_key(10), True, cuda)
    _, save = te.forward(qa, ca, pmask, sa)
    ref = te.backward(ct, qa, ca, pmask, save, sa).clone()
    _, save_a = te.forward(qa, ca, pmask, sa)
    te.forward(qb, cb, pmask, sb)
    got = te.backward(ct, qa, ca, pmask, save_a, sa)
    torch.cuda.synchronize()
    _same([ref], [got], "template embedding")


def test_design_step_save_survives(cuda):
    n, recycles = 64, 1
    print(f"design step fwd(A) fwd(B) bwd(A) n={n} recycles={recycles}", flush=True)
    depths = (1, 1, 2, 2)
    rng = np.random.default_rng(75)
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths[0], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths[1], rng),
           "main": {},
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    for b in range(depths[2]):
        prm["main"].update(bparams.init_block_params(b, rng, gates="random", ln="random"))
    prm["post"].update({f"const/{k}": v for k, v in bparams.init_residue_tables(rng).items()})
    dirs = [weights_dir(prm[k], f"survive_ds_{k}") for k in ("emb", "tpl", "extra", "main", "post")]
    step = ops.DesignStepSeq(*dirs, depths=depths)
    T = lambda a: torch.as_tensor(a, device=cuda)
    flags = np.ones(n, np.uint8)
    flags[: n // 2] = 2  # the first chain is the template (its MSA row joins the stack)
    ids = [T(np.arange(n, dtype=np.float32)), T(np.repeat([1, 2], n // 2).astype(np.float32)),
           T(np.repeat([1, 2], n // 2).astype(np.float32)), T(np.ones(n, np.float32))]
    seq_mask = T(np.ones(n, np.float32))
    sc = T(np.array([0.9, 0.1, 1.0, 1.0], np.float32))
    iasym = T(np.repeat([0, 1], n // 2).astype(np.int32))
    tpl37 = T((8 * rng.standard_normal((n, 37, 3))).astype(np.float32))
    tplm37 = T(np.ones((n, 37), np.float32))
    act_const = T((0.5 * rng.standard_normal((n, n, 64))).astype(np.float32))

    def seeds(base):
        return torch.tensor([[0, base + i, 1] for i in range(4 * (recycles + 1))],
                            dtype=torch.int64).to(torch.uint32).to(cuda)

    la = T(rng.standard_normal((n, 20)).astype(np.float32))
    lb = T(rng.standard_normal((n, 20)).astype(np.float32))
    cts = [T(rng.standard_normal(sh).astype(np.float32))
           for sh in ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))]
    conf_cts = [T(rng.standard_normal(sh).astype(np.float32))
                for sh in ((n,), (n, n), (1,), (1,), (n,), (n,))]
    ct37 = T(rng.standard_normal((n, 37, 3)).astype(np.float32))

    def fwd(logits, sd, save):
        step.forward(logits, T(flags), sc, ids, seq_mask, act_const=act_const, seeds=sd, save=save,
                     interface_asym=iasym, recycles=recycles, atom37=True, tpl_atoms37=tpl37,
                     tpl_mask37=tplm37)

    def bwd(logits, save):
        return step.backward(cts, logits, T(flags), sc, seq_mask, save, interface_asym=iasym,
                             conf_cts=conf_cts, d_atom37=ct37)

    nb = step.save_bytes(n)
    save_a = torch.empty(nb, dtype=torch.uint8, device=cuda)
    save_b = torch.empty(nb, dtype=torch.uint8, device=cuda)
    fwd(la, seeds(100), save_a)
    ref = bwd(la, save_a).clone()
    fwd(la, seeds(100), save_a)
    fwd(lb, seeds(200), save_b)
    got = bwd(la, save_a)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    _same([ref], [got], "design step")
