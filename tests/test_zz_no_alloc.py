"""The allocation-free triangle-attention forward (bc2n_triattn_fwd_noalloc)
through the C ABI: on two calls in a row, the second with a smaller N, its
pair output and save-set equal bc2n_triattn_fwd's bit for bit, the device's
free memory does not move across the calls, and an N beyond the static
scratch is refused with a clear error before any launch."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import lib, ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import random_mask, weights_dir

pytestmark = pytest.mark.gpu
NAME = "triangle_attention_ending_node"


def _ptr(t):
    return None if t is None else t.data_ptr()


def test_triattn_fwd_noalloc_matches_and_allocates_nothing(cuda):
    print("triattn_fwd_noalloc n=64 then n=32", flush=True)
    rng = np.random.default_rng(77)
    prm = bparams.init_block_params(0, rng, modules=[NAME], gates="random", ln="random")
    wdir = weights_dir(prm, "noalloc")
    prefix = f"param/block0/{NAME}/"
    mod = ops.TriangleAttention(wdir, prefix, per_column=True)
    L = lib()
    cases = []
    for n in (64, 32):
        pair = torch.as_tensor(rng.standard_normal((n, n, 128)).astype(np.float32), device=cuda)
        mask = torch.as_tensor(random_mask(n, 0.1, rng)[0], device=cuda)
        tbl = torch.as_tensor(af2.dropout_table(J.prng_key(n), 0.25, n, 128), device=cuda)
        ref_out, ref_save = mod.forward(pair, mask, tbl)  # also makes the weights resident
        out = torch.full_like(pair, float("nan"))
        save = torch.zeros_like(ref_save)
        cases.append((n, pair, mask, tbl, ref_out, ref_save, out, save))
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    stream = torch.cuda.current_stream().cuda_stream
    for n, pair, mask, tbl, _, _, out, save in cases:
        rc = L.bc2n_triattn_fwd_noalloc(stream, wdir.encode(), prefix.encode(), 1, n, _ptr(pair),
                                        _ptr(mask), _ptr(tbl), _ptr(out), _ptr(save))
        assert rc == 0, L.bc2n_last_error()
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    for n, _, _, _, ref_out, ref_save, out, save in cases:
        assert torch.equal(out, ref_out), f"pair output differs at n={n}"
        assert torch.equal(save, ref_save), f"save-set differs at n={n}"
    assert free1 == free0, (free0, free1)
    # beyond the static scratch: refused on the host, before any launch
    # (the operands are real buffers of the right size all the same)
    n = 288
    pair = torch.zeros(n, n, 128, device=cuda)
    mask = torch.ones(n, n, device=cuda)
    out = torch.empty_like(pair)
    save = torch.empty(mod.save_bytes(n), dtype=torch.uint8, device=cuda)
    rc = L.bc2n_triattn_fwd_noalloc(stream, wdir.encode(), prefix.encode(), 1, n, _ptr(pair),
                                    _ptr(mask), None, _ptr(out), _ptr(save))
    assert rc != 0
    assert b"static scratch" in L.bc2n_last_error()
