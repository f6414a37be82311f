"""The boundary's allocation contract through the C ABI (the reference's
prealloc entry points, native/ffi.cu:835-937, and its detached save=0
forward): after bc2n_*_prealloc, forward and backward calls at the prealloc'd
shapes leave the device's free memory unchanged; a detached forward equals
the saving forward bit for bit, writes no save-set and uses one block's
scratch (< 1 GB at L=224 against the 26 GB save-set)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import lib, ops, params as bparams
from oracle import jax_prng as J
from tests.helpers import random_mask, weights_dir

pytestmark = pytest.mark.gpu


def _free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0]


def _warm_torch_cache(nbytes):
    """Leave a cached block in torch's allocator so that the wrappers' own
    output tensors come from it, not from new device allocations: the free
    memory then moves only if the library allocates."""
    x = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    # tensors of <= 1 MB come from torch's small-block pool (2 MiB segments)
    small = [torch.empty(1 << 20, dtype=torch.uint8, device="cuda") for _ in range(32)]
    del x, small


@pytest.mark.timeout(600)
def test_stack_prealloc_and_detached_forward_L224(cuda):
    n, depth = 224, 48
    print(f"stack prealloc + detached forward n={n} depth={depth}", flush=True)
    rng = np.random.default_rng(2)
    evo, _, _ = bparams.init_trunk_params(rng, depth=depth, extra_depth=0, tpl_depth=0)
    st = ops.EvoformerStack(weights_dir(evo, "boundary_main"), depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    pair = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    msa = T(rng.standard_normal((1, n, 256)).astype(np.float32))
    pmask, m1 = random_mask(n, 0.1, rng)
    pmask, mmask = T(pmask), T(m1[None].copy())
    ct_pair, ct_msa = torch.randn_like(pair), torch.randn_like(msa)
    seed = ops.seed_tensor(J.prng_key(5), True, cuda)
    det_bytes, save_bytes = st.detached_bytes(n, 1), st.save_bytes(n, 1)
    print(f"  detached scratch {det_bytes / 1e9:.3f} GB, save-set {save_bytes / 1e9:.2f} GB",
          flush=True)
    assert det_bytes < 1e9 < save_bytes
    slots = lib().bc2n_save_slots_probe(st.dir, depth, n, 1, 0)
    assert slots > 0 and slots * n * n * 128 * 2 >= save_bytes
    save = torch.empty(save_bytes, dtype=torch.uint8, device=cuda)
    outs = [torch.empty_like(pair), torch.empty_like(msa), torch.empty_like(pair),
            torch.empty_like(msa)]
    st.prealloc(n, 1)
    _warm_torch_cache(256 << 20)
    f0 = _free()
    pd, md, none = st.forward(pair, msa, pmask, mmask, seed, detached=True, pair_out=outs[0],
                              msa_out=outs[1])
    assert none is None
    f1 = _free()
    po, mo, _ = st.forward(pair, msa, pmask, mmask, seed, save=save, pair_out=outs[2],
                           msa_out=outs[3])
    dp, dm = st.backward(ct_pair, ct_msa, pmask, mmask, save, seed)
    f2 = _free()
    print(f"  free memory across detached fwd: {f0 - f1} B; across fwd+bwd: {f1 - f2} B",
          flush=True)
    assert torch.equal(pd, po) and torch.equal(md, mo)
    assert torch.isfinite(dp).all() and torch.isfinite(dm).all()
    assert f1 == f0 and f2 == f1, (f0, f1, f2)


def test_component_preallocs_hold_memory(cuda):
    n = 64
    print(f"template / structure-module / template-embedding prealloc n={n}", flush=True)
    rng = np.random.default_rng(3)
    L = lib()
    tpl = {}
    for b in range(2):
        tpl.update(bparams.init_template_block_params(b, rng))
    d_tpl = weights_dir(tpl, "boundary_tpl")
    te = bparams.init_template_embedding_params(2, rng)
    d_te = weights_dir(te, "boundary_te")
    post = bparams.init_structure_heads_params(rng)
    post.update({f"const/{k}": v for k, v in bparams.init_residue_tables(rng).items()})
    d_post = weights_dir(post, "boundary_post")
    assert L.bc2n_tplstack_prealloc(n, 2, d_tpl.encode()) == 0, L.bc2n_last_error()
    assert L.bc2n_tplembed_prealloc(n, 2, d_te.encode()) == 0, L.bc2n_last_error()
    assert L.bc2n_sm_prealloc(n, 8, d_post.encode()) == 0, L.bc2n_last_error()
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask = T(random_mask(n, 0.1, rng)[0])
    seed = ops.seed_tensor(J.prng_key(9), True, cuda)
    # every buffer the calls take from torch, allocated before the first reading
    ts = ops.TemplatePairStack(d_tpl, 2)
    x64 = T(rng.standard_normal((n, n, 64)).astype(np.float32))
    s_ts = torch.empty(ts.save_bytes(n), dtype=torch.uint8, device=cuda)
    o_ts = torch.empty_like(x64)
    emb = ops.TemplateEmbedding(d_te, 2)
    q = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    s_te = torch.empty(emb.save_bytes(n), dtype=torch.uint8, device=cuda)
    sh = ops.StructureHeads(d_post, 8)
    single = T(rng.standard_normal((n, 384)).astype(np.float32))
    seq_mask = torch.ones(n, device=cuda)
    aatype = T(rng.integers(0, 20, n).astype(np.float32))
    _warm_torch_cache(256 << 20)
    f0 = _free()
    ts.forward(x64, pmask, seed, out=o_ts, save=s_ts)
    ts.backward(torch.ones_like(x64), pmask, s_ts, seed)
    out_te, _ = emb.forward(q, x64, pmask, seed, save=s_te)
    emb.backward(torch.ones_like(q), q, x64, pmask, s_te, seed)
    outs, s_sh = sh.forward(single, q, seq_mask, aatype, seed)
    sh.backward([torch.ones_like(o) for o in outs], single, q, seq_mask, aatype, s_sh)
    f1 = _free()
    print(f"  free memory moved by {f0 - f1} B", flush=True)
    assert f1 == f0, (f0, f1)
