"""Deep-stack reference runs on the CPU: the oracle's blocks (oracle/af2.py)
chained over a whole stack with per-block recompute, so that a 48-block
forward+backward at L=224 fits in host memory.

The forward keeps only each block's input carries; the backward re-runs one
block at a time under autograd from its saved input and pulls the running
cotangent through it.  Autograd of the oracle's block is the reference's VJP,
so the result equals autograd of the whole stack (layer_stack.py:66-204 scan,
modules_multimer.py:610-668) up to float rounding."""
import torch

from oracle import af2


def stack_forward(block, carries, keys):
    """block(b, *carries, key) -> tuple of carries.  Returns the list of every
    block's input carries plus the stack output (len(keys) + 1 entries)."""
    xs = [tuple(c.detach() for c in carries)]
    with torch.no_grad():
        for b, k in enumerate(keys):
            xs.append(tuple(block(b, *xs[-1], k)))
    return xs


def stack_backward(block, xs, keys, cts, progress=None):
    """Cotangents of the stack inputs from those of its outputs, one block at
    a time from the carries stack_forward kept (consumed as it goes)."""
    g = tuple(cts)
    for b in reversed(range(len(keys))):
        inp = tuple(t.detach().clone().requires_grad_(True) for t in xs[b])
        out = block(b, *inp, keys[b])
        g = torch.autograd.grad(out, inp, g)
        xs[b + 1] = None
        if progress is not None:
            progress(b)
    return g


def evoformer_block(params, pair_mask, msa_mask, use_dropout, dtype):
    def f(b, msa, pair, key):
        return af2.evoformer_iteration(msa, pair, msa_mask, pair_mask, params, f"param/block{b}/",
                                       key, use_dropout, dtype=dtype)
    return f


def pair_only_block(params, pair_mask, use_dropout, dtype):
    def f(b, pair, key):
        return (af2.pair_only_iteration(pair, pair_mask, params, f"param/block{b}/", key,
                                        use_dropout, dtype=dtype),)
    return f


def template_block(params, pair_mask, use_dropout, dtype):
    def f(b, act, key):
        return (af2.template_iteration(act, pair_mask, params, f"param/block{b}/", key, use_dropout,
                                       dtype=dtype),)
    return f
