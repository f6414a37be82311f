"""torch-tensor wrappers over the C ABI (device memory and streams only).

These mirror the reference's module interface (a module object built from a
weights directory + name prefix, forward -> (output, save), backward from the
save-set) so tests and benchmarks read like the reference's own module gates
(native/triattn.cu:51-75).  All arithmetic happens in libbc2n.so.
"""
import ctypes

import torch

from . import check, lib


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("bc2n ops take device tensors")
    if not t.is_contiguous():
        raise ValueError("bc2n ops take contiguous tensors")
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _f32(t, shape, name):
    if t.dtype != torch.float32 or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected float32 {tuple(shape)}, got {t.dtype} {tuple(t.shape)}")


class TriangleAttention:
    """modules.py TriangleAttention + dropout_wrapper, starting node
    (per_column=False) or ending node (per_column=True)."""

    def __init__(self, weights_dir, prefix, per_column, c=128, heads=4):
        self.dir = weights_dir.encode()
        self.prefix = prefix.encode()
        self.per_column = int(bool(per_column))
        self.c, self.h = c, heads

    def save_bytes(self, n):
        return lib().bc2n_triattn_save_bytes(n, self.c, self.h)

    def forward(self, pair, mask, drop_tbl=None, out=None, save=None):
        n = pair.shape[0]
        _f32(pair, (n, n, self.c), "pair")
        _f32(mask, (n, n), "pair_mask")
        if out is None:
            out = torch.empty_like(pair)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=pair.device)
        check(lib().bc2n_triattn_fwd(_stream(), self.dir, self.prefix, self.per_column, n,
                                     _ptr(pair), _ptr(mask), _ptr(drop_tbl), _ptr(out),
                                     _ptr(save)))
        return out, save

    def backward(self, pair, mask, drop_tbl, save, dout, din=None):
        n = pair.shape[0]
        _f32(dout, (n, n, self.c), "dpair_out")
        if din is None:
            din = torch.empty_like(dout)
        check(lib().bc2n_triattn_bwd(_stream(), self.dir, self.prefix, self.per_column, n,
                                     _ptr(pair), _ptr(mask), _ptr(drop_tbl), _ptr(save),
                                     _ptr(dout), _ptr(din)))
        return din


class TriangleMultiplication:
    """modules.py TriangleMultiplication (fused projections) + dropout_wrapper,
    outgoing or incoming."""

    def __init__(self, weights_dir, prefix, outgoing, c=128, hidden=128):
        self.dir = weights_dir.encode()
        self.prefix = prefix.encode()
        self.outgoing = int(bool(outgoing))
        self.c, self.i = c, hidden

    def save_bytes(self, n):
        return lib().bc2n_trimul_save_bytes(n, self.c, self.i)

    def forward(self, pair, mask, drop_tbl=None, out=None, save=None):
        n = pair.shape[0]
        _f32(pair, (n, n, self.c), "pair")
        _f32(mask, (n, n), "pair_mask")
        if out is None:
            out = torch.empty_like(pair)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=pair.device)
        check(lib().bc2n_trimul_fwd(_stream(), self.dir, self.prefix, self.outgoing, n,
                                    _ptr(pair), _ptr(mask), _ptr(drop_tbl), _ptr(out),
                                    _ptr(save)))
        return out, save

    def backward(self, pair, mask, drop_tbl, save, dout, din=None):
        n = pair.shape[0]
        _f32(dout, (n, n, self.c), "dpair_out")
        if din is None:
            din = torch.empty_like(dout)
        check(lib().bc2n_trimul_bwd(_stream(), self.dir, self.prefix, self.outgoing, n,
                                    _ptr(pair), _ptr(mask), _ptr(drop_tbl), _ptr(save),
                                    _ptr(dout), _ptr(din)))
        return din


def dropout_table(rows, channels, key, rate, device="cuda"):
    """[rows, channels] keep/keep_rate table from a JAX key (k0, k1)."""
    tbl = torch.empty(rows, channels, dtype=torch.float32, device=device)
    check(lib().bc2n_dropout_table(_stream(), _ptr(tbl), rows, channels,
                                   int(key[0]), int(key[1]), float(rate)))
    return tbl


def bernoulli_bits(n, key, rate, device="cuda"):
    out = torch.empty(n, dtype=torch.uint8, device=device)
    check(lib().bc2n_bernoulli_bits(_stream(), _ptr(out), n, int(key[0]), int(key[1]),
                                    float(rate)))
    return out


def stack_keys(seed, depth, device="cuda"):
    """[depth, 9, 2] uint32 module keys from the stack key (k0, k1)."""
    s = torch.tensor([int(seed[0]), int(seed[1])], dtype=torch.int64).to(torch.uint32)
    s = s.to(device)
    out = torch.empty(depth * 9 * 2, dtype=torch.uint32, device=device)
    check(lib().bc2n_stack_keys(_stream(), _ptr(s), depth, _ptr(out)))
    return out.view(depth, 9, 2)


def probe_gemm(a_bf16, b_bf16):
    """C = A . B^T (bf16 in, f32 out) through the library's MFMA GEMM."""
    m, k = a_bf16.shape
    n = b_bf16.shape[0]
    c = torch.empty(m, n, dtype=torch.float32, device=a_bf16.device)
    check(lib().bc2n_probe_gemm(_stream(), m, n, k, _ptr(a_bf16), _ptr(b_bf16), _ptr(c)))
    return c


def probe_layernorm(x, gamma, beta, fast=False):
    m, c = x.shape
    y = torch.empty(m, c, dtype=torch.bfloat16, device=x.device)
    mean = torch.empty(m, dtype=torch.float32, device=x.device)
    rstd = torch.empty(m, dtype=torch.float32, device=x.device)
    check(lib().bc2n_probe_layernorm(_stream(), m, c, _ptr(x), _ptr(gamma), _ptr(beta),
                                     int(fast), _ptr(y), _ptr(mean), _ptr(rstd)))
    return y, mean, rstd
