"""torch-tensor wrappers over the C ABI (device memory and streams only).

These mirror the reference's module interface (a module object built from a
weights directory + name prefix, forward -> (output, save), backward from the
save-set) so tests and benchmarks read like the reference's own module gates
(native/triattn.cu:51-75).  All arithmetic happens in libbc2n.so.
"""
import contextlib
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


class Transition:
    """modules.py Transition + dropout_wrapper over act [B, N, C] (pair:
    B = N; MSA: B = S)."""

    def __init__(self, weights_dir, prefix, c, factor=4):
        self.dir, self.prefix, self.c, self.f = weights_dir.encode(), prefix.encode(), c, factor

    def forward(self, act, drop_tbl=None):
        b, n, c = act.shape
        rows = b * n
        out = torch.empty_like(act)
        save = torch.empty(lib().bc2n_transition_save_bytes(rows, c, self.f), dtype=torch.uint8,
                           device=act.device)
        check(lib().bc2n_transition_fwd(_stream(), self.dir, self.prefix, rows, n, _ptr(act),
                                        _ptr(drop_tbl), _ptr(out), _ptr(save)))
        return out, save

    def backward(self, act, drop_tbl, save, dout):
        b, n, c = act.shape
        din = torch.empty_like(dout)
        check(lib().bc2n_transition_bwd(_stream(), self.dir, self.prefix, b * n, n, _ptr(act),
                                        _ptr(drop_tbl), _ptr(save), _ptr(dout), _ptr(din)))
        return din


class OuterProductMean:
    """modules.py OuterProductMean added into the pair (dropout_wrapper)."""

    def __init__(self, weights_dir, prefix, outer=32, c_z=128):
        self.dir, self.prefix, self.o, self.cz = weights_dir.encode(), prefix.encode(), outer, c_z

    def forward(self, msa, msa_mask, pair, drop_tbl=None):
        s, n, _ = msa.shape
        out = torch.empty_like(pair)
        save = torch.empty(lib().bc2n_opm_save_bytes(s, n, self.o, self.cz), dtype=torch.uint8,
                           device=msa.device)
        check(lib().bc2n_opm_fwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa), _ptr(msa_mask),
                                 _ptr(pair), _ptr(drop_tbl), _ptr(out), _ptr(save)))
        return out, save

    def backward(self, msa, msa_mask, drop_tbl, save, dpair, dmsa_out=None):
        s, n, _ = msa.shape
        if dmsa_out is None:
            dmsa_out = torch.zeros_like(msa)
        dmsa = torch.empty_like(msa)
        check(lib().bc2n_opm_bwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa), _ptr(msa_mask),
                                 _ptr(drop_tbl), _ptr(save), _ptr(dpair), _ptr(dmsa_out),
                                 _ptr(dmsa)))
        return dmsa


class MSARowAttentionWithPairBias:
    def __init__(self, weights_dir, prefix, c_m=256, heads=8):
        self.dir, self.prefix, self.cm, self.h = weights_dir.encode(), prefix.encode(), c_m, heads

    def forward(self, msa, msa_mask, pair, drop_tbl=None):
        s, n, _ = msa.shape
        out = torch.empty_like(msa)
        save = torch.empty(lib().bc2n_msarow_save_bytes(s, n, self.cm, self.h), dtype=torch.uint8,
                           device=msa.device)
        check(lib().bc2n_msarow_fwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                    _ptr(msa_mask), _ptr(pair), _ptr(drop_tbl), _ptr(out),
                                    _ptr(save)))
        return out, save

    def backward(self, msa, msa_mask, pair, drop_tbl, save, dout, dpair=None):
        s, n, _ = msa.shape
        din = torch.empty_like(dout)
        if dpair is None:
            dpair = torch.zeros_like(pair)
        check(lib().bc2n_msarow_bwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                    _ptr(msa_mask), _ptr(pair), _ptr(drop_tbl), _ptr(save),
                                    _ptr(dout), _ptr(din), _ptr(dpair)))
        return din, dpair


class MSAColumnGlobalAttention:
    """The extra-MSA stack's column module (modules.py:619-672), f32."""

    def __init__(self, weights_dir, prefix):
        self.dir, self.prefix = weights_dir.encode(), prefix.encode()

    def forward(self, msa, msa_mask, drop_tbl=None):
        s, n, _ = msa.shape
        out = torch.empty_like(msa)
        nb = lib().bc2n_msaglobal_save_bytes(self.dir, self.prefix, s, n)
        if nb == 0:
            check(1)
        save = torch.empty(nb, dtype=torch.uint8, device=msa.device)
        check(lib().bc2n_msaglobal_fwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                       _ptr(msa_mask), _ptr(drop_tbl), _ptr(out), _ptr(save)))
        return out, save

    def backward(self, msa, msa_mask, drop_tbl, save, dout):
        s, n, _ = msa.shape
        din = torch.empty_like(dout)
        check(lib().bc2n_msaglobal_bwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                       _ptr(msa_mask), _ptr(drop_tbl), _ptr(save), _ptr(dout),
                                       _ptr(din)))
        return din


class MSAColumnAttention:
    def __init__(self, weights_dir, prefix, c_m=256, heads=8):
        self.dir, self.prefix, self.cm, self.h = weights_dir.encode(), prefix.encode(), c_m, heads

    def forward(self, msa, msa_mask, drop_tbl=None):
        s, n, _ = msa.shape
        out = torch.empty_like(msa)
        save = torch.empty(lib().bc2n_msacol_save_bytes(s, n, self.cm, self.h), dtype=torch.uint8,
                           device=msa.device)
        check(lib().bc2n_msacol_fwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                    _ptr(msa_mask), _ptr(drop_tbl), _ptr(out), _ptr(save)))
        return out, save

    def backward(self, msa, msa_mask, drop_tbl, save, dout):
        s, n, _ = msa.shape
        din = torch.empty_like(dout)
        check(lib().bc2n_msacol_bwd(_stream(), self.dir, self.prefix, s, n, _ptr(msa),
                                    _ptr(msa_mask), _ptr(drop_tbl), _ptr(save), _ptr(dout),
                                    _ptr(din)))
        return din


def _seed_len(seed):
    """Length of a seed operand as the C ABI takes it: the tensor's own word
    count (u32[3] = [k0, k1, enabled], or the reference caller's u32[2] =
    [bits, enabled]); 3 when there is none (dropout off)."""
    if seed is None:
        return 3
    if seed.dtype not in (torch.uint32, torch.int32) or seed.numel() not in (2, 3):
        raise ValueError("seed must be u32[3] [k0, k1, enabled] or u32[2] [bits, enabled]")
    return seed.numel()


def seed_tensor(key, enabled=True, device="cuda"):
    """The stack's seed operand u32[3] = [k0, k1, enabled] (key_data of the
    stack's JAX key plus the use_dropout flag)."""
    t = torch.tensor([int(key[0]), int(key[1]), int(bool(enabled))], dtype=torch.int64)
    return t.to(torch.uint32).to(device)


def bits_seed_tensor(bits, enabled=True, device="cuda"):
    """The reference caller's seed operand u32[2] = [bits, enabled]
    (modules_multimer.py:660-667: jax.random.bits of the stack's subkey and
    use_dropout); the library keys the stack with PRNGKey(bits) = (0, bits)."""
    t = torch.tensor([int(bits) & 0xFFFFFFFF, int(bool(enabled))], dtype=torch.int64)
    return t.to(torch.uint32).to(device)


class EvoformerStack:
    """The drop-in for the reference's native_evoformer_fwd/bwd FFI pair
    (native/ffi.cu:942-982): `depth` Evoformer blocks from a weights
    directory, pure forward/backward with the save-set crossing as data."""

    def __init__(self, weights_dir, depth, pair_only=False, c_m=256):
        self.dir, self.depth, self.pair_only, self.cm = weights_dir.encode(), depth, pair_only, c_m

    def save_bytes(self, n, s):
        b = lib().bc2n_evoformer_save_bytes(self.dir, n, s, self.depth, int(self.pair_only))
        if b == 0:
            check(1)
        return b

    def detached_bytes(self, n, s):
        b = lib().bc2n_evoformer_detached_bytes(self.dir, n, s, self.depth, int(self.pair_only))
        if b == 0:
            check(1)
        return b

    def prealloc(self, n, s, dropout=True):
        """Upload the weights and grow every scratch buffer the calls at
        these shapes use (native_stack_prealloc's counterpart)."""
        check(lib().bc2n_stack_prealloc(n, s, self.depth, self.dir, int(self.pair_only), 1,
                                        int(dropout)))

    def forward(self, pair, msa, pair_mask, msa_mask, seed=None, dropout=True, save=None,
                pair_out=None, msa_out=None, detached=False):
        """detached=True: the save=0 forward (no backward follows); no
        save-set is written and None is returned for it."""
        n = pair.shape[0]
        s, _, cm = msa.shape
        if pair_out is None:
            pair_out = torch.empty_like(pair)
        if msa_out is None:
            msa_out = torch.empty_like(msa)
        if save is None and not detached:
            save = torch.empty(self.save_bytes(n, s), dtype=torch.uint8, device=pair.device)
        seed_len = _seed_len(seed)
        check(lib().bc2n_evoformer_fwd(_stream(), _ptr(pair), _ptr(msa), _ptr(pair_mask),
                                       _ptr(msa_mask), _ptr(seed), seed_len, n, s, cm,
                                       self.depth, 0 if detached else 1, int(self.pair_only), 0,
                                       1, int(dropout), self.dir, _ptr(pair_out), _ptr(msa_out),
                                       None if detached else _ptr(save), None))
        return pair_out, msa_out, (None if detached else save)

    def backward(self, ct_pair, ct_msa, pair_mask, msa_mask, save, seed=None, dropout=True):
        n = ct_pair.shape[0]
        s, _, cm = ct_msa.shape
        dpair = torch.empty_like(ct_pair)
        dmsa = torch.empty_like(ct_msa)
        seed_len = _seed_len(seed)
        check(lib().bc2n_evoformer_bwd(_stream(), _ptr(ct_pair), _ptr(ct_msa), _ptr(pair_mask),
                                       _ptr(msa_mask), _ptr(save), None, _ptr(seed),
                                       seed_len, n, s, cm, self.depth,
                                       int(self.pair_only), 0, 1, int(dropout), self.dir,
                                       _ptr(dpair), _ptr(dmsa)))
        return dpair, dmsa


SAVE_POLICIES = {"auto": 0, "full": 1, "replay": 2}


@contextlib.contextmanager
def save_policy(name):
    """Run the enclosed stack calls under a save policy (bc2n_set_save_policy):
    'auto' (the replay tier only where the full save-set would not fit),
    'full' or 'replay'; the previous policy is restored on exit."""
    old = lib().bc2n_set_save_policy(SAVE_POLICIES[name])
    if old < 0:
        check(1)
    try:
        yield
    finally:
        lib().bc2n_set_save_policy(old)


@contextlib.contextmanager
def msa_overlap(on):
    """Run the enclosed stack calls with the MSA side of each Evoformer block
    on the library's second stream (True, the default) or on the caller's
    stream (False); the previous setting is restored on exit."""
    old = lib().bc2n_set_msa_overlap(int(bool(on)))
    try:
        yield
    finally:
        lib().bc2n_set_msa_overlap(old)


class TemplatePairStack:
    """The drop-in for TemplatePairStackFwd/Bwd (native/ffi.cu:983-1008)."""

    def __init__(self, weights_dir, depth):
        self.dir, self.depth = weights_dir.encode(), depth

    def save_bytes(self, n):
        b = lib().bc2n_tplstack_save_bytes(self.dir, n, self.depth)
        if b == 0:
            check(1)
        return b

    def forward(self, pair, pair_mask, seed=None, dropout=True, out=None, save=None):
        n = pair.shape[0]
        if out is None:
            out = torch.empty_like(pair)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=pair.device)
        seed_len = _seed_len(seed)
        check(lib().bc2n_tplstack_fwd(_stream(), _ptr(pair), _ptr(pair_mask), _ptr(seed),
                                      seed_len, n, self.depth, int(dropout), self.dir, _ptr(out),
                                      _ptr(save)))
        return out, save

    def backward(self, ct, pair_mask, save, seed=None, dropout=True):
        n = ct.shape[0]
        dpair = torch.empty_like(ct)
        seed_len = _seed_len(seed)
        check(lib().bc2n_tplstack_bwd(_stream(), _ptr(ct), _ptr(pair_mask), _ptr(save),
                                      _ptr(seed), seed_len, n, self.depth, int(dropout), self.dir,
                                      _ptr(dpair)))
        return dpair


class TemplateEmbedding:
    """The drop-in for TemplateEmbeddingFwd/Bwd (native/ffi.cu:1072-1098): one
    template, the eight constant feature projections summed into act_const;
    query [N,N,128] -> out [N,N,128] through the template pair stack."""

    def __init__(self, weights_dir, depth):
        self.dir, self.depth = weights_dir.encode(), depth

    def save_bytes(self, n):
        b = lib().bc2n_tplembed_save_bytes(self.dir, n, self.depth)
        if b == 0:
            check(1)
        return b

    def forward(self, query, act_const, pair_mask, seed=None, dropout=True, out=None, save=None):
        n = query.shape[0]
        if out is None:
            out = torch.empty_like(query)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=query.device)
        seed_len = _seed_len(seed)
        check(lib().bc2n_tplembed_fwd(_stream(), _ptr(query), _ptr(act_const), _ptr(pair_mask),
                                      _ptr(seed), seed_len, n, self.depth, int(dropout), self.dir,
                                      _ptr(out), _ptr(save)))
        return out, save

    def backward(self, ct, query, act_const, pair_mask, save, seed=None, dropout=True):
        n = ct.shape[0]
        dquery = torch.empty_like(ct)
        seed_len = _seed_len(seed)
        check(lib().bc2n_tplembed_bwd(_stream(), _ptr(ct), _ptr(query), _ptr(act_const),
                                      _ptr(pair_mask), _ptr(save), _ptr(seed), seed_len, n,
                                      self.depth, int(dropout), self.dir, _ptr(dquery)))
        return dquery


class Embedder:
    """The drop-in for EmbedderFwd/Bwd (native/ffi.cu:1046-1071): target_feat
    [N,21] (padded), msa_feat [S,N,49] and the four id features [N] ->
    msa [S,N,256], pair [N,N,128]; backward (dmsa, dpair, target_feat) ->
    (dtarget_feat [N,21], dmsa_feat [S,N,49]).  All f32, no save-set."""

    def __init__(self, weights_dir):
        self.dir = weights_dir.encode()

    def forward(self, target_feat, msa_feat, residue_index, asym_id, entity_id, sym_id,
                offset=None, msa=None, pair=None):
        n, s = target_feat.shape[0], msa_feat.shape[0]
        dev = target_feat.device
        if msa is None:
            msa = torch.empty(s, n, 256, dtype=torch.float32, device=dev)
        if pair is None:
            pair = torch.empty(n, n, 128, dtype=torch.float32, device=dev)
        check(lib().bc2n_embedder_fwd(_stream(), _ptr(target_feat), _ptr(msa_feat),
                                      _ptr(residue_index), _ptr(asym_id), _ptr(entity_id),
                                      _ptr(sym_id), _ptr(offset), n, s, self.dir, _ptr(msa),
                                      _ptr(pair)))
        return msa, pair

    def backward(self, dmsa, dpair, target_feat):
        s, n = dmsa.shape[0], dmsa.shape[1]
        dtf = torch.empty(n, 21, dtype=torch.float32, device=dmsa.device)
        dmf = torch.empty(s, n, 49, dtype=torch.float32, device=dmsa.device)
        check(lib().bc2n_embedder_bwd(_stream(), _ptr(dmsa), _ptr(dpair), _ptr(target_feat), n, s,
                                      self.dir, _ptr(dtf), _ptr(dmf)))
        return dtf, dmf


class Fold:
    """The structure module's fold iterations (IPA + transition + rigid
    update, the part of StructureHeadsFwd/Bwd before the sidechain,
    native/ffi.cu:1009-1044), f32."""

    def __init__(self, weights_dir, depth=8):
        self.dir, self.depth = weights_dir.encode(), depth

    def save_bytes(self, n):
        b = lib().bc2n_fold_save_bytes(self.dir, n, self.depth)
        if b == 0:
            check(1)
        return b

    def forward(self, single, pair, seq_mask, seed=None, dropout=True, save=None):
        """-> (act [N,384], traj [depth,N,3,4], save)"""
        n = single.shape[0]
        act = torch.empty_like(single)
        traj = torch.empty(self.depth, n, 3, 4, dtype=torch.float32, device=single.device)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=single.device)
        seed_len = _seed_len(seed)
        check(lib().bc2n_fold_fwd(_stream(), _ptr(single), _ptr(pair), _ptr(seq_mask), _ptr(seed),
                                  seed_len, n, self.depth, int(dropout), self.dir, _ptr(act),
                                  _ptr(traj), _ptr(save)))
        return act, traj, save

    def backward(self, d_act, d_traj, single, pair, seq_mask, save, dropout=True):
        """-> (dsingle, dpair); d_act / d_traj may be None."""
        n = single.shape[0]
        dsingle = torch.empty_like(single)
        dpair = torch.empty_like(pair)
        check(lib().bc2n_fold_bwd(_stream(), _ptr(d_act), _ptr(d_traj), _ptr(single), _ptr(pair),
                                  _ptr(seq_mask), _ptr(save), n, self.depth, int(dropout),
                                  self.dir, _ptr(dsingle), _ptr(dpair)))
        return dsingle, dpair


class StructureHeads:
    """The drop-in for StructureHeadsFwd/Bwd (native/ffi.cu:1009-1044): fold
    iterations, the last iteration's sidechain (atom14) and the distogram,
    PAE, pLDDT and experimentally-resolved heads, f32."""

    def __init__(self, weights_dir, depth=8):
        self.dir, self.depth = weights_dir.encode(), depth

    def save_bytes(self, n):
        b = lib().bc2n_structure_heads_save_bytes(self.dir, n, self.depth)
        if b == 0:
            check(1)
        return b

    def forward(self, single, pair, seq_mask, aatype, seed=None, dropout=True, save=None):
        """-> ((atom14 [N,14,3], distogram [N,N,64], pae [N,N,64], plddt [N,50],
        expres [N,37]), save)"""
        n, dev = single.shape[0], single.device
        outs = tuple(torch.empty(*sh, dtype=torch.float32, device=dev)
                     for sh in ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37)))
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=dev)
        seed_len = _seed_len(seed)
        check(lib().bc2n_structure_heads_fwd(_stream(), _ptr(single), _ptr(pair), _ptr(seq_mask),
                                             _ptr(aatype), _ptr(seed), seed_len, n, self.depth,
                                             int(dropout), self.dir, *map(_ptr, outs), _ptr(save)))
        return outs, save

    def backward(self, cts, single, pair, seq_mask, aatype, save, dropout=True):
        """cts = (d_atom14, d_distogram, d_pae, d_plddt, d_expres), each may
        be None -> (dsingle, dpair)"""
        n = single.shape[0]
        dsingle, dpair = torch.empty_like(single), torch.empty_like(pair)
        check(lib().bc2n_structure_heads_bwd(_stream(), _ptr(single), _ptr(pair), _ptr(seq_mask),
                                             _ptr(aatype), *map(_ptr, cts), _ptr(save), n,
                                             self.depth, int(dropout), self.dir, _ptr(dsingle),
                                             _ptr(dpair)))
        return dsingle, dpair


class DesignStep:
    """The trunk of one design step in one call (bc2n_design_step_*):
    embedder, template embedding (when act_const is given), extra-MSA stack
    (pair only), main stack, single projection, structure module and heads;
    backward to d(target_feat), d(msa_feat)."""

    def __init__(self, emb_dir, tpl_dir, extra_dir, main_dir, post_dir, depths=(2, 4, 48, 8)):
        self.dirs = [d.encode() for d in (emb_dir, tpl_dir, extra_dir, main_dir, post_dir)]
        self.depths = tuple(int(d) for d in depths)  # template, extra, main, fold

    def save_bytes(self, n, s):
        b = lib().bc2n_design_step_save_bytes(*self.dirs, n, s, *self.depths)
        if b == 0:
            check(1)
        return b

    def forward(self, target_feat, msa_feat, ids, seq_mask, aatype, act_const=None, offset=None,
                seeds=None, dropout=True, save=None, recycles=0):
        """ids = (residue_index, asym_id, entity_id, sym_id); seeds
        u32[recycles + 1][4][3] (per pass the keys of the template, extra,
        main and structure-module stacks) -> ((atom14, distogram, pae, plddt,
        expres), save) of the last of recycles + 1 passes"""
        n, s, dev = target_feat.shape[0], msa_feat.shape[0], target_feat.device
        _check_seeds(seeds, dropout, recycles)
        outs = tuple(torch.empty(*sh, dtype=torch.float32, device=dev)
                     for sh in ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37)))
        if save is None:
            save = torch.empty(self.save_bytes(n, s), dtype=torch.uint8, device=dev)
        check(lib().bc2n_design_step_fwd(_stream(), _ptr(target_feat), _ptr(msa_feat),
                                         *map(_ptr, ids), _ptr(offset), _ptr(seq_mask),
                                         _ptr(act_const), _ptr(aatype), _ptr(seeds), n, s,
                                         *self.depths, int(dropout), int(recycles), *self.dirs,
                                         *map(_ptr, outs), _ptr(save)))
        return outs, save

    def backward(self, cts, target_feat, seq_mask, aatype, save, with_template=True,
                 dropout=True, msa_rows=1):
        n = target_feat.shape[0]
        dtf = torch.empty_like(target_feat)
        dmf = torch.empty(msa_rows, n, 49, dtype=torch.float32, device=target_feat.device)
        check(lib().bc2n_design_step_bwd(_stream(), _ptr(target_feat), _ptr(seq_mask),
                                         _ptr(aatype), int(with_template), *map(_ptr, cts),
                                         _ptr(save), n, msa_rows, *self.depths, int(dropout),
                                         *self.dirs, _ptr(dtf), _ptr(dmf)))
        return dtf, dmf


def _check_seeds(seeds, dropout, recycles):
    """A design step's seeds hold (recycles + 1) x 4 keys of 3 words."""
    if recycles < 0:
        raise ValueError("recycles must be >= 0")
    if dropout and (seeds is None or seeds.numel() != (recycles + 1) * 12):
        raise ValueError(f"dropout needs seeds u32[{recycles + 1}][4][3]")


OMITTED_HALF = -5000.0  # half of BindCraft's omitted-acid logit (-1e4)


class SeqFeat:
    """Design sequence features (bc2n_seqfeat_*, the reference's GlueSeqFeat /
    GlueSeqFeatBwd): logits [N, 20], flags u8 [N] (bit 0 = designed), bias [20]
    or None; scalars = (softmax_weight, one_hot_weight, temperature,
    logit_scale) as floats, or a device tensor [4] that overrides them."""

    def __init__(self, scalars, aa_bias=None, omitted_half=OMITTED_HALF):
        self.dev_scalars = scalars if torch.is_tensor(scalars) else None
        self.vals = (1.0, 0.0, 1.0, 1.0) if self.dev_scalars is not None else \
            tuple(float(x) for x in scalars)
        self.bias, self.omitted = aa_bias, float(omitted_half)

    def forward(self, logits, flags):
        n = logits.shape[0]
        feat, prof = torch.empty_like(logits), torch.empty_like(logits)
        check(lib().bc2n_seqfeat_fwd(_stream(), _ptr(logits), _ptr(flags), _ptr(self.bias),
                                     *self.vals, self.omitted, _ptr(self.dev_scalars), n,
                                     _ptr(feat), _ptr(prof)))
        return feat, prof

    def backward(self, logits, flags, d_feat, d_prof):
        n = logits.shape[0]
        d = torch.empty_like(logits)
        check(lib().bc2n_seqfeat_bwd(_stream(), _ptr(logits), _ptr(flags), _ptr(self.bias),
                                     _ptr(d_feat), _ptr(d_prof), *self.vals, self.omitted,
                                     _ptr(self.dev_scalars), n, _ptr(d)))
        return d


def design_inputs(feat, prof):
    """(feat, prof) [N, 20] -> target_feat [N, 21], msa_feat [1, N, 49], aatype [N] (float)."""
    n, dev = feat.shape[0], feat.device
    tf = torch.empty(n, 21, dtype=torch.float32, device=dev)
    mf = torch.empty(1, n, 49, dtype=torch.float32, device=dev)
    aat = torch.empty(n, dtype=torch.float32, device=dev)
    check(lib().bc2n_design_inputs_fwd(_stream(), _ptr(feat), _ptr(prof), n, _ptr(tf), _ptr(mf),
                                       _ptr(aat)))
    return tf, mf, aat


def design_inputs_backward(d_target_feat, d_msa_feat):
    n, dev = d_target_feat.shape[0], d_target_feat.device
    d_feat = torch.empty(n, 20, dtype=torch.float32, device=dev)
    d_prof = torch.empty(n, 20, dtype=torch.float32, device=dev)
    check(lib().bc2n_design_inputs_bwd(_stream(), _ptr(d_target_feat), _ptr(d_msa_feat), n,
                                       _ptr(d_feat), _ptr(d_prof)))
    return d_feat, d_prof


def _length(t):
    """A runtime length operand: None, or an i32 tensor of one element on the
    device (never read on the host)."""
    if t is None:
        return None
    if t.dtype != torch.int32 or t.numel() != 1 or not t.is_cuda:
        raise ValueError("length must be a one-element int32 tensor on the device")
    return t


class DesignStepSeq(DesignStep):
    """The one-call design step from the designed logits
    (bc2n_design_step_seq_*): sequence features -> trunk inputs -> the step;
    backward to d(logits).  scalars: device tensor [4] (softmax_weight,
    one_hot_weight, temperature, logit_scale)."""

    def save_bytes(self, n, s=1):
        b = lib().bc2n_design_step_seq_save_bytes(*self.dirs, n, *self.depths)
        if b == 0:
            check(1)
        return b

    def forward(self, logits, flags, scalars, ids, seq_mask, aa_bias=None, act_const=None,
                offset=None, seeds=None, dropout=True, save=None, omitted_half=OMITTED_HALF,
                interface_asym=None, recycles=0, atom37=False, tpl_atoms37=None,
                tpl_mask37=None, length=None, cyclic_mode=None, flexibility=0.0,
                initial_atom_pos=False):
        """-> ((atom14, distogram, pae, plddt, expres), save), plus the confidence
        metrics (plddt, pae, ptm, iptm, iptm_per_residue, expres_ca) as a third
        element when interface_asym (i32 [N]) is given.  With atom37=True (or
        template atoms tpl_atoms37 [N,37,3] / tpl_mask37 [N,37], which align
        them) a fourth element (atom37 [N,37,3], exists mask [N,37]) follows
        the third (None without interface_asym).  length: an i32 device tensor
        [1] holding the runtime length (rows at or past it are padding), or
        None for all N rows.  cyclic_mode ('distance', 'direction',
        'neighbours' or None = `offset` as given) builds the offset feature
        from the ids and the CYCLIC flag (bit 6); flexibility is the target
        flexibility of the template row; initial_atom_pos starts the structure
        module from tpl_atoms37 (needs a cyclic_mode, as the reference packs
        it into that attribute)."""
        modes = ("distance", "direction", "neighbours")
        cmode = -1 if cyclic_mode is None else modes.index(cyclic_mode)
        if initial_atom_pos:
            if cyclic_mode is None:
                raise ValueError("initial_atom_pos goes with a cyclic_mode")
            cmode |= 4
        n, dev = logits.shape[0], logits.device
        _check_seeds(seeds, dropout, recycles)
        e = lambda *sh: torch.empty(*sh, dtype=torch.float32, device=dev)
        outs = (e(n, 14, 3), e(n, n, 64), e(n, n, 64), e(n, 50), e(n, 37))
        conf = (e(n), e(n, n), e(1), e(1), e(n), e(n)) if interface_asym is not None else (None,) * 6
        want37 = atom37 or tpl_atoms37 is not None
        a37 = (e(n, 37, 3), e(n, 37)) if want37 else (None, None)
        if save is None:
            save = torch.empty(self.save_bytes(n), dtype=torch.uint8, device=dev)
        check(lib().bc2n_design_step_seq_fwd(_stream(), _ptr(logits), _ptr(flags), _ptr(aa_bias),
                                             _ptr(scalars), float(omitted_half), *map(_ptr, ids),
                                             _ptr(offset), _ptr(seq_mask), _ptr(act_const),
                                             _ptr(seeds), n, _ptr(_length(length)),
                                             *self.depths, int(dropout),
                                             int(recycles), cmode, float(flexibility),
                                             *self.dirs, *map(_ptr, outs),
                                             _ptr(tpl_atoms37), _ptr(tpl_mask37),
                                             *map(_ptr, a37), _ptr(interface_asym),
                                             *map(_ptr, conf), _ptr(save)))
        if want37:
            return outs, save, (conf if interface_asym is not None else None), a37
        if interface_asym is None:
            return outs, save
        return outs, save, conf

    def backward(self, cts, logits, flags, scalars, seq_mask, save, aa_bias=None,
                 with_template=True, dropout=True, omitted_half=OMITTED_HALF,
                 interface_asym=None, conf_cts=(None,) * 6, d_atom37=None, length=None):
        n = logits.shape[0]
        d = torch.empty_like(logits)
        check(lib().bc2n_design_step_seq_bwd(_stream(), _ptr(logits), _ptr(flags), _ptr(aa_bias),
                                             _ptr(scalars), float(omitted_half), _ptr(seq_mask),
                                             int(with_template), *map(_ptr, cts),
                                             _ptr(d_atom37), _ptr(interface_asym),
                                             *map(_ptr, conf_cts),
                                             _ptr(save), n, _ptr(_length(length)),
                                             *self.depths, int(dropout), *self.dirs, _ptr(d)))
        return d


class Confidence:
    """pLDDT, symmetrised PAE, pTM, ipTM (+ per residue) and the CA
    experimentally-resolved probability from the head logits
    (bc2n_confidence_*)."""

    def forward(self, plddt_logits, pae_logits, expres_logits, seq_mask, interface_asym):
        n, dev = plddt_logits.shape[0], plddt_logits.device
        e = lambda *sh: torch.empty(*sh, dtype=torch.float32, device=dev)
        outs = (e(n), e(n, n), e(1), e(1), e(n), e(n))
        save = torch.empty(lib().bc2n_confidence_save_bytes(n), dtype=torch.uint8, device=dev)
        check(lib().bc2n_confidence_fwd(_stream(), _ptr(plddt_logits), _ptr(pae_logits),
                                        _ptr(expres_logits), _ptr(seq_mask), _ptr(interface_asym),
                                        n, *map(_ptr, outs), _ptr(save)))
        return outs, save

    def backward(self, cts, plddt_logits, pae_logits, expres_logits, seq_mask, interface_asym,
                 save):
        """cts = (d_plddt, d_pae, d_ptm, d_iptm, d_iptm_per_residue, d_expres_ca), any None"""
        n = plddt_logits.shape[0]
        d = (torch.empty_like(plddt_logits), torch.empty_like(pae_logits),
             torch.empty_like(expres_logits))
        check(lib().bc2n_confidence_bwd(_stream(), _ptr(plddt_logits), _ptr(pae_logits),
                                        _ptr(expres_logits), _ptr(seq_mask), _ptr(interface_asym),
                                        _ptr(save), *map(_ptr, cts), n, *map(_ptr, d)))
        return d


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


def probe_gemm(a_f16, b_f16):
    """C = A . B^T (binary16 in, f32 out) through the library's MFMA GEMM."""
    if a_f16.dtype != torch.float16 or b_f16.dtype != torch.float16:
        raise TypeError("probe_gemm: operands must be float16 (the GEMM's operand format)")
    m, k = a_f16.shape
    n = b_f16.shape[0]
    c = torch.empty(m, n, dtype=torch.float32, device=a_f16.device)
    check(lib().bc2n_probe_gemm(_stream(), m, n, k, _ptr(a_f16), _ptr(b_f16), _ptr(c)))
    return c


def probe_mfma(form, blocks, iters, device="cuda"):
    """Launch the MFMA issue-rate probe (form 0: 16x16x32 f16, 1: 16x16x16
    f16, 2: 32x32x16 f16, 3: 16x16x32 bf16); returns (FLOPs launched, output
    tensor)."""
    out = torch.empty(blocks * 256, dtype=torch.float32, device=device)
    flops = lib().bc2n_probe_mfma(_stream(), int(form), int(blocks), int(iters), _ptr(out))
    if flops < 0:
        check(1)
    return flops, out


def probe_layernorm(x, gamma, beta, fast=False):
    m, c = x.shape
    y = torch.empty(m, c, dtype=torch.float16, device=x.device)
    mean = torch.empty(m, dtype=torch.float32, device=x.device)
    rstd = torch.empty(m, dtype=torch.float32, device=x.device)
    check(lib().bc2n_probe_layernorm(_stream(), m, c, _ptr(x), _ptr(gamma), _ptr(beta),
                                     int(fast), _ptr(y), _ptr(mean), _ptr(rstd)))
    return y, mean, rstd


def probe_gemm_f32(A, B, C, M, N, K, batch, a_strides, b_strides, c_strides):
    """C[b,m,n] = sum_k A[.] B[.] with element strides (test hook)."""
    check(lib().bc2n_probe_gemm_f32(_stream(), M, N, K, batch, _ptr(A), *a_strides, _ptr(B),
                                    *b_strides, _ptr(C), *c_strides))
    return C


def probe_recycle(emb_dir, pair, msa0, aatype=None, prev_atom14=None, prev_pair=None,
                  prev_msa0=None):
    """pair [N,N,128] and msa0 [N,256] (f32, in place) += the design step's
    recycle terms of the previous state (bc2n_probe_recycle); no previous
    state = the first pass."""
    n = pair.shape[0]
    check(lib().bc2n_probe_recycle(_stream(), n, emb_dir.encode(), _ptr(aatype), _ptr(prev_atom14),
                                   _ptr(prev_pair), _ptr(prev_msa0), _ptr(pair), _ptr(msa0)))
    return pair, msa0

