"""CPU restatement of the reference's JAX AlphaFold2 trunk (fp64/fp32 torch).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product never routes
through this module.

Every function follows one function of the reference, cited by file:line
(paths under bindcraft/af/alphafold/model/ unless noted), einsum by einsum, so
autograd of this code is the reference's VJP.  Parameters are a flat dict in
the weights-manifest naming ``param/block{b}/<module>/<param>`` (the names
bindcraft/af/native.py:205-226 writes), values numpy float32 arrays.

Pinning (tests/test_oracle_*.py): LayerNorm/Linear/attention against textbook
closed forms and torch.nn.functional at fp64; attention against a pure-Python
loop on tiny inputs; triangle attention ending == starting on the transposed
pair; incoming == outgoing with swapped operands; OPM against its direct
4-index sum and the mask==0 constant; S=1 column attention against its
softmax==1 closed form; global attention against a pure-Python loop, its
S=1 closed form and its fully-masked-column closed form; the pair-only extra
block against the full extra-MSA iteration on a zero mask; the recycle
terms' distogram against a loop over the squared breaks, and the first-pass
terms against their closed form (bias + offsets); Kabsch against scipy's
weighted Rotation.align_vectors, an exact rigid motion (recovered exactly), a
mirror image (a proper rotation still) and no weights (the identity); the
atom37 gather against a loop; the dihedral against constructed quadruples of
known torsion and the chi mask against a loop; gradients against central
finite differences.
"""
import contextlib
import math

import numpy as np
import torch
import torch.utils.checkpoint

from . import jax_prng

LOGIT_CLIP = 1e8  # bindcraft/af/accel.py:6

_RECOMPUTE = [False]


@contextlib.contextmanager
def block_recompute():
    """Within this context every stack block that runs under autograd keeps
    only its input (activation checkpointing) and is run again in the
    backward, so a deep stack at L = 224 fits in host memory.  Autograd of
    the recomputed block is the same VJP (dropout keys are explicit, nothing
    draws from torch's generator), so the results do not change."""
    old = _RECOMPUTE[0]
    _RECOMPUTE[0] = True
    try:
        yield
    finally:
        _RECOMPUTE[0] = old


def _run_block(fn, *args):
    if _RECOMPUTE[0] and torch.is_grad_enabled():
        return torch.utils.checkpoint.checkpoint(fn, *args, use_reentrant=False)
    return fn(*args)


class Params:
    """Prefix view over a flat parameter dict, converting to torch."""

    def __init__(self, params, prefix, dtype=torch.float64):
        self.params, self.prefix, self.dtype = params, prefix, dtype

    def __call__(self, name):
        return torch.as_tensor(np.asarray(self.params[self.prefix + name]), dtype=self.dtype)

    def sub(self, name):
        return Params(self.params, self.prefix + name, self.dtype)


def layer_norm(x, scale, offset, fast=False, eps=1e-5):
    """common_modules.py:127-183 (haiku LayerNorm); fast=True is the
    use_fast_variance form of modules.py:909-919."""
    mean = x.mean(-1, keepdim=True)
    if fast:
        var = (x * x).mean(-1, keepdim=True) - mean * mean
    else:
        var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return (x - mean) * (torch.rsqrt(var + eps) * scale) + offset


def linear(x, p):
    """common_modules.py:52-118 (Linear: '...c,cd->...d' + bias)."""
    return torch.einsum("...c,cd->...d", x, p("weights")) + p("bias")


def attention(q_data, m_data, bias, nonbatched_bias, p, gating=True):
    """modules.py:313-400 (Attention) with accel.py:13-22 (_attend_stock:
    logits + bias + nonbatched bias, clipped to +-LOGIT_CLIP, softmax)."""
    qw, kw, vw = p("attention/query_w"), p("attention/key_w"), p("attention/value_w")
    key_dim = qw.shape[-1]
    q = torch.einsum("bqa,ahc->bqhc", q_data, qw) * key_dim ** (-0.5)
    k = torch.einsum("bka,ahc->bkhc", m_data, kw)
    v = torch.einsum("bka,ahc->bkhc", m_data, vw)
    logits = torch.einsum("bqhc,bkhc->bhqk", q, k) + bias
    if nonbatched_bias is not None:
        logits = logits + nonbatched_bias[None]
    logits = torch.clamp(logits, -LOGIT_CLIP, LOGIT_CLIP)
    weights = torch.softmax(logits, dim=-1)
    wa = torch.einsum("bhqk,bkhc->bqhc", weights, v)
    if gating:
        gate = torch.einsum("bqc,chv->bqhv", q_data, p("attention/gating_w")) + p("attention/gating_b")
        wa = wa * torch.sigmoid(gate)
    return torch.einsum("bqhc,hco->bqo", wa, p("attention/output_w")) + p("attention/output_b")


def global_attention(q_data, m_data, q_mask, p, gating=True):
    """modules.py:403-497 (GlobalAttention)."""
    qw, kw, vw = p("attention/query_w"), p("attention/key_w"), p("attention/value_w")
    key_dim = qw.shape[-1]
    v = torch.einsum("bka,ac->bkc", m_data, vw)
    q_avg = (q_mask * q_data).sum(1) / (q_mask.sum(1) + 1e-10)  # utils.mask_mean
    q = torch.einsum("ba,ahc->bhc", q_avg, qw) * key_dim ** (-0.5)
    k = torch.einsum("bka,ac->bkc", m_data, kw)
    bias = 1e9 * (q_mask[:, None, :, 0] - 1.0)
    logits = torch.einsum("bhc,bkc->bhk", q, k) + bias
    weights = torch.softmax(logits, dim=-1)
    wa = torch.einsum("bhk,bkc->bhc", weights, v)
    ow, ob = p("attention/output_w"), p("attention/output_b")
    if gating:
        gate = torch.sigmoid(torch.einsum("bqc,chv->bqhv", q_data, p("attention/gating_w"))
                             + p("attention/gating_b"))
        wa = wa[:, None] * gate
        return torch.einsum("bqhc,hco->bqo", wa, ow) + ob
    return (torch.einsum("bhc,hco->bo", wa, ow) + ob)[:, None]


def triangle_attention(pair, mask, p, per_column):
    """modules.py:675-734 (TriangleAttention); per_column = ending node."""
    if per_column:
        pair = pair.transpose(0, 1)
        mask = mask.transpose(0, 1)
    bias = (1e9 * (mask - 1.0))[:, None, None, :]
    x = layer_norm(pair, p("query_norm/scale"), p("query_norm/offset"))
    nb = torch.einsum("qkc,ch->hqk", x, p("feat_2d_weights"))
    out = attention(x, x, bias, nb, p)
    if per_column:
        out = out.transpose(0, 1)
    return out


def triangle_attention_vjp(pair, mask, p, per_column, dout, scale=None, rows=64):
    """(delta, d pair) of triangle_attention(pair) * scale under the
    cotangent dout, with the attention evaluated `rows` batch rows at a time.
    The same functions as triangle_attention (layer_norm, the feat_2d bias
    einsum, attention), composed the same way; the batch rows of `attention`
    are independent, so each chunk's VJP is taken on its own and the
    cotangents of the shared LayerNorm output and pair bias are summed before
    one VJP through them.  Peak memory is one chunk's [rows, H, N, N] logits
    instead of the whole [N, H, N, N] graph (17 GB a copy at N = 1024 in
    f32).  scale: the dropout table [N, C] (applied per row, or per column
    for the ending node), or None."""
    x0 = pair.detach().requires_grad_(True)
    sc = None if scale is None else (scale[:, None] if per_column else scale[None])
    dz = dout if sc is None else dout * sc
    xp, mk = x0, mask
    if per_column:
        xp, mk, dz = x0.transpose(0, 1), mask.transpose(0, 1), dz.transpose(0, 1)
    x = layer_norm(xp, p("query_norm/scale"), p("query_norm/offset"))
    nb = torch.einsum("qkc,ch->hqk", x, p("feat_2d_weights"))
    bias = (1e9 * (mk - 1.0))[:, None, None, :]
    xd, nbd = x.detach().requires_grad_(True), nb.detach().requires_grad_(True)
    out = torch.empty_like(dz)
    for r0 in range(0, xd.shape[0], rows):
        sl = slice(r0, r0 + rows)
        o = attention(xd[sl], xd[sl], bias[sl], nbd, p)
        out[sl] = o.detach()
        torch.autograd.backward(o, dz[sl])
    torch.autograd.backward((x, nb), (xd.grad, nbd.grad))
    if per_column:
        out = out.transpose(0, 1)
    return (out if sc is None else out * sc), x0.grad


def triangle_multiplication(pair, mask, p, outgoing):
    """modules.py:1044-1088 (_fused_triangle_multiplication); equations
    'ikc,jkc->ijc' (outgoing) / 'kjc,kic->ijc' (incoming), config.py:440-453."""
    m = mask[..., None]
    x = layer_norm(pair, p("left_norm_input/scale"), p("left_norm_input/offset"), fast=True)
    proj = m * linear(x, p.sub("projection/"))
    proj = proj * torch.sigmoid(linear(x, p.sub("gate/")))
    nI = proj.shape[-1] // 2
    left, right = proj[..., :nI], proj[..., nI:]
    eq = "ikc,jkc->ijc" if outgoing else "kjc,kic->ijc"
    act = torch.einsum(eq, left, right)
    act = layer_norm(act, p("center_norm/scale"), p("center_norm/offset"), fast=True)
    act = linear(act, p.sub("output_projection/"))
    return act * torch.sigmoid(linear(x, p.sub("gating_linear/")))


def transition(act, mask, p):
    """modules.py:252-305 (Transition): LN -> Linear+relu -> Linear."""
    x = layer_norm(act, p("input_layer_norm/scale"), p("input_layer_norm/offset"))
    h = torch.relu(linear(x, p.sub("transition1/")))
    return linear(h, p.sub("transition2/"))


def outer_product_mean(msa, mask, p):
    """modules.py:1128-1212 (OuterProductMean)."""
    m = mask[..., None]
    x = layer_norm(msa, p("layer_norm_input/scale"), p("layer_norm_input/offset"))
    left = m * linear(x, p.sub("left_projection/"))
    right = m * linear(x, p.sub("right_projection/"))
    act = torch.einsum("abc,ade->bdce", left, right)
    act = torch.einsum("bdce,cef->bdf", act, p("output_w")) + p("output_b")
    norm = torch.einsum("abc,adc->bdc", m, m)
    return act / (1e-3 + norm)


def msa_row_attention(msa, msa_mask, pair, p):
    """modules.py:500-563 (MSARowAttentionWithPairBias)."""
    bias = (1e9 * (msa_mask - 1.0))[:, None, None, :]
    x = layer_norm(msa, p("query_norm/scale"), p("query_norm/offset"))
    z = layer_norm(pair, p("feat_2d_norm/scale"), p("feat_2d_norm/offset"))
    nb = torch.einsum("qkc,ch->hqk", z, p("feat_2d_weights"))
    return attention(x, x, bias, nb, p)


def msa_column_attention(msa, msa_mask, p):
    """modules.py:566-616 (MSAColumnAttention)."""
    msa = msa.transpose(0, 1)
    msa_mask = msa_mask.transpose(0, 1)
    bias = (1e9 * (msa_mask - 1.0))[:, None, None, :]
    x = layer_norm(msa, p("query_norm/scale"), p("query_norm/offset"))
    return attention(x, x, bias, None, p).transpose(0, 1)


def msa_column_global_attention(msa, msa_mask, p):
    """modules.py:619-672 (MSAColumnGlobalAttention)."""
    msa = msa.transpose(0, 1)
    msa_mask = msa_mask.transpose(0, 1)
    x = layer_norm(msa, p("query_norm/scale"), p("query_norm/offset"))
    out = global_attention(x, x, msa_mask[..., None], p)
    return out.transpose(0, 1)


# ------------------------------------------------------------------ dropout

def dropout_keep(key, rate, shape):
    """The keep mask of apply_dropout (modules.py:37-44) as float64 0/1."""
    keep = jax_prng.bernoulli(key, jax_prng.keep_rate(rate), shape)
    return torch.as_tensor(keep.astype(np.float64))


def apply_dropout(tensor, key, rate, broadcast_dim):
    """modules.py:37-44: keep * tensor / keep_rate, keep shared over
    broadcast_dim."""
    if rate == 0.0 or key is None:
        return tensor
    shape = list(tensor.shape)
    if broadcast_dim is not None:
        shape[broadcast_dim] = 1
    keep = dropout_keep(key, rate, tuple(shape)).to(tensor.dtype)
    return keep * tensor / float(jax_prng.keep_rate(rate))


def dropout_table(key, rate, rows, channels):
    """The [rows, C] scale table the native path consumes for a shared mask
    of shape (1, rows, C) or (rows, 1, C): keep / keep_rate."""
    keep = jax_prng.bernoulli(key, jax_prng.keep_rate(rate), (rows, channels))
    return keep.astype(np.float32) / np.float32(jax_prng.keep_rate(rate))


# Module configuration of the multimer Evoformer (config.py:386-460):
# (name, dropout rate, orientation).
EVO_MODULES = (
    ("outer_product_mean", 0.0, "per_row"),
    ("msa_row_attention_with_pair_bias", 0.15, "per_row"),
    ("msa_column_attention", 0.0, "per_column"),
    ("msa_transition", 0.0, "per_row"),
    ("triangle_multiplication_outgoing", 0.25, "per_row"),
    ("triangle_multiplication_incoming", 0.25, "per_row"),
    ("triangle_attention_starting_node", 0.25, "per_row"),
    ("triangle_attention_ending_node", 0.25, "per_column"),
    ("pair_transition", 0.0, "per_row"),
)


def dropout_wrapper(residual, output_act, key, rate, orientation, use_dropout):
    """modules.py:46-76: output_act + apply_dropout(residual) with the shared
    mask's broadcast dim 0 for 'per_row' and 1 for 'per_column'."""
    bd = 0 if orientation == "per_row" else 1
    r = rate if use_dropout else 0.0
    return output_act + apply_dropout(residual, key, r, bd)


def evoformer_iteration(msa, pair, msa_mask, pair_mask, params, prefix, key,
                        use_dropout, is_extra_msa=False, dtype=torch.float64):
    """modules.py:1278-1391 (EvoformerIteration) with outer_product_mean.first
    (config.py:414).  `key` is the block's SafeKey value: split into 10, keys
    1..9 go to the 9 modules in order (modules.py:1308-1309)."""
    P = Params(params, prefix, dtype)
    sub = jax_prng.split(key, 10)[1:] if key is not None else [None] * 9
    cfg = {n: (r, o) for n, r, o in EVO_MODULES}

    def wrap(name, residual, out_act, k):
        r, o = cfg[name]
        return dropout_wrapper(residual, out_act, k, r, o, use_dropout)

    pair = wrap("outer_product_mean",
                outer_product_mean(msa, msa_mask, P.sub("outer_product_mean/")), pair, sub[0])
    msa = wrap("msa_row_attention_with_pair_bias",
               msa_row_attention(msa, msa_mask, pair, P.sub("msa_row_attention_with_pair_bias/")),
               msa, sub[1])
    if is_extra_msa:
        col = msa_column_global_attention(msa, msa_mask, P.sub("msa_column_global_attention/"))
    else:
        col = msa_column_attention(msa, msa_mask, P.sub("msa_column_attention/"))
    msa = wrap("msa_column_attention", col, msa, sub[2])
    msa = wrap("msa_transition", transition(msa, msa_mask, P.sub("msa_transition/")), msa, sub[3])
    pair = wrap("triangle_multiplication_outgoing",
                triangle_multiplication(pair, pair_mask, P.sub("triangle_multiplication_outgoing/"), True),
                pair, sub[4])
    pair = wrap("triangle_multiplication_incoming",
                triangle_multiplication(pair, pair_mask, P.sub("triangle_multiplication_incoming/"), False),
                pair, sub[5])
    pair = wrap("triangle_attention_starting_node",
                triangle_attention(pair, pair_mask, P.sub("triangle_attention_starting_node/"), False),
                pair, sub[6])
    pair = wrap("triangle_attention_ending_node",
                triangle_attention(pair, pair_mask, P.sub("triangle_attention_ending_node/"), True),
                pair, sub[7])
    pair = wrap("pair_transition", transition(pair, pair_mask, P.sub("pair_transition/")), pair, sub[8])
    return msa, pair


def pair_only_iteration(pair, pair_mask, params, prefix, key, use_dropout, dtype=torch.float64):
    """The pair track of an extra-MSA EvoformerIteration (modules.py:1278-1391)
    whose extra-MSA mask is all zero, as the design step runs it
    (bindcraft/af2.py:193; the reference's native pair-only stack,
    bindcraft/af/native.py:1131-1193): the outer product mean of a fully
    masked MSA is output_b / 1e-3 (left = right = 0, norm = 0) at dropout
    rate 0, the MSA modules never reach the pair again, and the five pair
    modules take keys 5..9 of the block key's split into 10."""
    P = Params(params, prefix, dtype)
    sub = jax_prng.split(key, 10)[1:] if key is not None else [None] * 9
    cfg = {n: (r, o) for n, r, o in EVO_MODULES}
    pair = pair + P("outer_product_mean/output_b") / 1e-3
    for i, name in enumerate(("triangle_multiplication_outgoing", "triangle_multiplication_incoming",
                              "triangle_attention_starting_node", "triangle_attention_ending_node",
                              "pair_transition")):
        p = P.sub(name + "/")
        if name.startswith("triangle_multiplication"):
            res = triangle_multiplication(pair, pair_mask, p, name.endswith("outgoing"))
        elif name.startswith("triangle_attention"):
            res = triangle_attention(pair, pair_mask, p, name.endswith("ending_node"))
        else:
            res = transition(pair, pair_mask, p)
        r, o = cfg[name]
        pair = dropout_wrapper(res, pair, sub[4 + i], r, o, use_dropout)
    return pair


def stack_block_keys(stack_key, depth):
    """The key each layer of a layer_stack scan hands its block
    (modules_multimer.py:622-641, :957-975): per layer (carry, sub) =
    split(carry); None entries when there is no key."""
    out, carry = [], stack_key
    for _ in range(depth):
        if carry is None:
            out.append(None)
            continue
        carry, sub = jax_prng.split(carry, 2)
        out.append(sub)
    return out


def evoformer_stack(msa, pair, msa_mask, pair_mask, params, depth, stack_key,
                    use_dropout, is_extra_msa=False, dtype=torch.float64):
    """modules_multimer.py:610-641 (layer_stack scan of evoformer_fn): per
    layer (carry, sub) = split(carry); the block gets `sub`."""
    carry = stack_key
    for b in range(depth):
        if carry is not None:
            carry, sub = jax_prng.split(carry, 2)
        else:
            sub = None
        msa, pair = _run_block(
            lambda m, z, b=b, sub=sub: evoformer_iteration(m, z, msa_mask, pair_mask, params,
                                                           f"param/block{b}/", sub, use_dropout,
                                                           is_extra_msa, dtype), msa, pair)
    return msa, pair


# Template pair stack (modules_multimer.py:1008-1077), rates/orientations of
# config.py template_pair_stack.
TPL_MODULES = (
    ("triangle_multiplication_outgoing", 0.25, "per_row"),
    ("triangle_multiplication_incoming", 0.25, "per_row"),
    ("triangle_attention_starting_node", 0.25, "per_row"),
    ("triangle_attention_ending_node", 0.25, "per_column"),
    ("pair_transition", 0.0, "per_row"),
)


def template_iteration(act, pair_mask, params, prefix, key, use_dropout, dtype=torch.float64):
    """modules_multimer.py:1017-1077 (TemplateEmbeddingIteration): the block
    key is split into 20; keys 1..5 go to the five modules in order."""
    P = Params(params, prefix, dtype)
    sub = jax_prng.split(key, 20)[1:6] if key is not None else [None] * 5
    for (name, rate, orient), k in zip(TPL_MODULES, sub):
        p = P.sub(name + "/")
        if name.startswith("triangle_multiplication"):
            res = triangle_multiplication(act, pair_mask, p, name.endswith("outgoing"))
        elif name.startswith("triangle_attention"):
            res = triangle_attention(act, pair_mask, p, name.endswith("ending_node"))
        else:
            res = transition(act, pair_mask, p)
        act = dropout_wrapper(res, act, k, rate, orient, use_dropout)
    return act


def template_stack(act, pair_mask, params, depth, stack_key, use_dropout, dtype=torch.float64):
    """modules_multimer.py:957-975 (layer_stack of template_iteration_fn)."""
    carry = stack_key
    for b in range(depth):
        if carry is not None:
            carry, sub = jax_prng.split(carry, 2)
        else:
            sub = None
        act = _run_block(lambda x, b=b, sub=sub: template_iteration(
            x, pair_mask, params, f"param/block{b}/", sub, use_dropout, dtype), act)
    return act


def template_embedding(query, act_const, pair_mask, params, depth, stack_key, use_dropout,
                       dtype=torch.float64):
    """modules_multimer.py:704-1005 (TemplateEmbedding) for one template with the
    eight constant feature projections already summed into `act_const`
    (:940-951, query_projection :922-940): the ninth feature is
    Linear(LN(query)) (query_embedding_norm, template_pair_embedding_8); the
    stack (:956-991) gets `stack_key`; then output_layer_norm (:1000-1005),
    the mean over num_templates = 1 and relu (:802-803), output_linear
    (:804-808)."""
    P = Params(params, "param/", dtype)
    q = layer_norm(query, P("query_embedding_norm/scale"), P("query_embedding_norm/offset"))
    act = act_const + linear(q, P.sub("template_pair_embedding_8/"))
    act = template_stack(act, pair_mask, params, depth, stack_key, use_dropout, dtype)
    act = layer_norm(act, P("output_layer_norm/scale"), P("output_layer_norm/offset"))
    return linear(torch.relu(act), P.sub("output_linear/"))


# -------------------------------------------------------------------- embedder
# modules_multimer.py:358-483 (multimer embedder; config.py:465-467:
# use_chain_relative, max_relative_chain 2, max_relative_idx 32).
MAX_RELATIVE_IDX = 32
MAX_RELATIVE_CHAIN = 2


def relative_encoding(residue_index, asym_id, entity_id, sym_id, p, offset=None,
                      dtype=torch.float64):
    """modules_multimer.py:358-435 (_relative_encoding, use_chain_relative):
    the concatenation of a 66-wide one-hot of the clipped offset (bin 65 =
    different chain), the same-entity flag and a 6-wide one-hot of the
    clipped sym_id difference (bin 5 = different entity), [N,N,73], through
    position_activations.  `offset` replaces residue_index[i] -
    residue_index[j] when given (:384-388).  Ids are integer-valued."""
    k, c = MAX_RELATIVE_IDX, MAX_RELATIVE_CHAIN
    ri, ai = torch.as_tensor(residue_index).long(), torch.as_tensor(asym_id).long()
    ei, si = torch.as_tensor(entity_id).long(), torch.as_tensor(sym_id).long()
    asym_same = ai[:, None] == ai[None, :]
    off = ri[:, None] - ri[None, :] if offset is None else torch.as_tensor(offset).long()
    clipped = torch.clamp(off + k, 0, 2 * k)
    final = torch.where(asym_same, clipped, torch.full_like(clipped, 2 * k + 1))
    rel_pos = torch.nn.functional.one_hot(final, 2 * k + 2).to(dtype)
    ent_same = ei[:, None] == ei[None, :]
    rel_sym = si[:, None] - si[None, :]
    clipped_chain = torch.clamp(rel_sym + c, 0, 2 * c)
    final_chain = torch.where(ent_same, clipped_chain, torch.full_like(clipped_chain, 2 * c + 1))
    rel_chain = torch.nn.functional.one_hot(final_chain, 2 * c + 2).to(dtype)
    feat = torch.cat([rel_pos, ent_same.to(dtype)[..., None], rel_chain], -1)
    return linear(feat, p)


def embedder(target_feat, msa_feat, residue_index, asym_id, entity_id, sym_id, params,
             offset=None, feature_mask=True, dtype=torch.float64):
    """modules_multimer.py:441-483 + :510-511 (the four input Linears and the
    relative encoding) on target_feat ALREADY padded to 21 columns (:450):
    msa = preprocess_1d(tf)[None] + preprocess_msa(msa_feat), pair =
    left_single(tf)[:, None] + right_single(tf)[None] + relative encoding.
    feature_mask zeroes preprocess_1d on rows whose target_feat sums to zero,
    as the reference's native embedder does (native/embed.cuh:22-25, 187-195,
    310); the JAX path (:476-478) has no such mask, and the two agree wherever
    no row sums to zero.  position_activations may sit under
    param/evoformer/~_relative_encoding/ (haiku's method scope) or param/."""
    P = Params(params, "param/", dtype)
    pre1d = linear(target_feat, P.sub("preprocess_1d/"))
    if feature_mask:
        pre1d = pre1d * (target_feat.sum(-1) != 0).to(dtype)[:, None]
    msa = pre1d[None] + linear(msa_feat, P.sub("preprocess_msa/"))
    left = linear(target_feat, P.sub("left_single/"))
    right = linear(target_feat, P.sub("right_single/"))
    scoped = "param/evoformer/~_relative_encoding/position_activations/"
    pos = Params(params, scoped if scoped + "weights" in params else "param/position_activations/",
                 dtype)
    pair = left[:, None] + right[None] + relative_encoding(residue_index, asym_id, entity_id,
                                                           sym_id, pos, offset, dtype)
    return msa, pair


# ------------------------------------------------------------ structure module
# folding_multimer.py (AF2 multimer structure module), config.py:578-600.
IPA_HEADS, IPA_SCALAR_QK, IPA_POINT_QK, IPA_SCALAR_V, IPA_POINT_V = 12, 16, 4, 16, 8
FOLD_DROPOUT = 0.1         # config.py:578
POSITION_SCALE = 20.0      # config.py:595


def _linear_nd(x, p, bias=True):
    """common_modules.Linear with a multi-dimensional output: weights
    [C, *out] flattened to [C, prod(out)], output reshaped back."""
    w = p("weights")
    out_shape = tuple(w.shape[1:])
    y = torch.einsum("...c,cd->...d", x, w.reshape(w.shape[0], -1))
    if bias and (p.prefix + "bias") in p.params:
        y = y + p("bias").reshape(-1)
    return y.reshape(*x.shape[:-1], *out_shape)


def quat_to_rot(w, x, y, z, eps=1e-6):
    """geometry/rotation_matrix.py:117-140 (from_quaternion, normalize=True):
    rows [[xx, xy, xz], [yx, yy, yz], [zx, zy, zz]]."""
    inv = torch.rsqrt(torch.clamp(w * w + x * x + y * y + z * z, min=eps))
    w, x, y, z = w * inv, x * inv, y * inv, z * inv
    r0 = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1)
    r1 = torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1)
    r2 = torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1)
    return torch.stack([r0, r1, r2], -2)


def point_projection(act, p, R, t, num_points):
    """folding_multimer.py:148-185: Linear(C -> H x 3P) split as
    [x(P) | y(P) | z(P)] per head, then to the global frame R p + t."""
    local = _linear_nd(act, p)                              # [N, H, 3P]
    P_ = num_points
    loc = torch.stack([local[..., :P_], local[..., P_:2 * P_], local[..., 2 * P_:]], -1)
    return torch.einsum("nij,nhpj->nhpi", R, loc) + t[:, None, None, :]


def invariant_point_attention(act, act_2d, mask, R, t, p, dist_eps=1e-8):
    """folding_multimer.py:188-371 (InvariantPointAttention)."""
    n = act.shape[0]
    raw = p("trainable_point_weights")
    point_w = math.sqrt(1.0 / (max(IPA_POINT_QK, 1) * 9.0 / 2)) * torch.logaddexp(
        raw, torch.zeros_like(raw))
    q_pt = point_projection(act, p.sub("q_point_projection/point_projection/"), R, t, IPA_POINT_QK)
    k_pt = point_projection(act, p.sub("k_point_projection/point_projection/"), R, t, IPA_POINT_QK)
    dist2 = ((q_pt[:, None] - k_pt[None]) ** 2).sum(-1)          # [q, k, H, P]
    logits = -0.5 * (point_w[:, None] * dist2).sum(-1)             # [q, k, H]
    q_s = _linear_nd(act, p.sub("q_scalar_projection/")) * math.sqrt(1.0 / IPA_SCALAR_QK)
    k_s = _linear_nd(act, p.sub("k_scalar_projection/"))
    logits = logits + torch.einsum("qhc,khc->qkh", q_s, k_s)
    logits = logits + linear(act_2d, p.sub("attention_2d/"))
    mask_2d = mask[:, None] * mask[None, :]
    logits = logits - 1e5 * (1.0 - mask_2d[..., None])
    logits = logits * math.sqrt(1.0 / 3)
    attn = torch.softmax(logits, dim=-2)
    v_s = _linear_nd(act, p.sub("v_scalar_projection/"))
    res_s = torch.einsum("qkh,khc->qhc", attn, v_s)
    v_pt = point_projection(act, p.sub("v_point_projection/point_projection/"), R, t, IPA_POINT_V)
    res_g = torch.einsum("qkh,khpi->qhpi", attn, v_pt)
    res_l = torch.einsum("nji,nhpj->nhpi", R, res_g - t[:, None, None, :])  # R^T (g - t)
    norms = torch.sqrt(torch.clamp((res_l ** 2).sum(-1), min=dist_eps ** 2))
    res_2d = torch.einsum("ijh,ijc->ihc", attn, act_2d)
    final = torch.cat([res_s.reshape(n, -1), res_l[..., 0].reshape(n, -1),
                       res_l[..., 1].reshape(n, -1), res_l[..., 2].reshape(n, -1),
                       norms.reshape(n, -1), res_2d.reshape(n, -1)], -1)
    return linear(final, p.sub("output_projection/"))


def fold_iteration(act, R, t, act_2d, mask, p, key, use_dropout):
    """folding_multimer.py:374-474 (FoldIteration, update_rigid=True) up to
    the rigid update; the sidechain (MultiRigidSidechain) is not part of it.
    The rotation carries gradient (the reference's stop_gradient is
    commented out, :467)."""
    act = act + invariant_point_attention(act, act_2d, mask, R, t,
                                          p.sub("invariant_point_attention/"))
    k1, k2 = jax_prng.split(key, 3)[1:3] if key is not None else (None, None)
    rate = FOLD_DROPOUT if use_dropout else 0.0
    act = apply_dropout(act, k1, rate, None)
    act = layer_norm(act, p("attention_layer_norm/scale"), p("attention_layer_norm/offset"))
    inp = act
    act = torch.relu(linear(act, p.sub("transition/")))
    act = torch.relu(linear(act, p.sub("transition_1/")))
    act = linear(act, p.sub("transition_2/")) + inp
    act = apply_dropout(act, k2, rate, None)
    act = layer_norm(act, p("transition_layer_norm/scale"), p("transition_layer_norm/offset"))
    flat = linear(act, p.sub("quat_rigid/rigid/"))                 # [N, 6]
    Ru = quat_to_rot(torch.ones_like(flat[:, 0]), flat[:, 0], flat[:, 1], flat[:, 2])
    t_new = torch.einsum("nij,nj->ni", R, flat[:, 3:6]) + t
    return act, R @ Ru, t_new


def frames_from_atoms(pos37):
    """folding_multimer.py:508-515 (initial_atom_pos) with
    all_atom_multimer.py:943-966 and geometry/rotation_matrix.py:79-99:
    R's columns e0 = unit(C - CA), e1 = unit((N - CA) - ((N - CA).e0) e0),
    e2 = e0 x e1, unit() clipping the norm at 1e-6 (an all-zero residue
    gives the zero matrix); t = CA / POSITION_SCALE."""
    pos = torch.as_tensor(pos37)

    def unit(v):
        return v / torch.sqrt(torch.clamp((v * v).sum(-1, keepdim=True), min=1e-12))

    n, ca, c = pos[:, 0], pos[:, 1], pos[:, 2]
    e0 = unit(c - ca)
    e1 = n - ca
    e1 = unit(e1 - (e1 * e0).sum(-1, keepdim=True) * e0)
    e2 = torch.linalg.cross(e0, e1)
    return torch.stack([e0, e1, e2], -1), ca / POSITION_SCALE


def fold(single, pair, mask, params, depth, key, use_dropout, dtype=torch.float64,
         init_pos=None):
    """folding_multimer.py:476-548 (generate_monomer_rigids): LN + initial
    projection, identity frames (or, given initial atom positions init_pos
    [N,37,3], frames_from_atoms of them), LN(pair), then `depth`
    FoldIterations sharing one set of weights with per-layer keys
    split(key, depth).  Returns the final act and the trajectory
    [depth, N, 3, 4] = [R | POSITION_SCALE * t] (StructureModule 'traj')."""
    P = Params(params, "param/", dtype)
    act = layer_norm(single, P("single_layer_norm/scale"), P("single_layer_norm/offset"))
    act = linear(act, P.sub("initial_projection/"))
    act_2d = layer_norm(pair, P("pair_layer_norm/scale"), P("pair_layer_norm/offset"))
    n = single.shape[0]
    if init_pos is None:
        R = torch.eye(3, dtype=single.dtype).expand(n, 3, 3)
        t = torch.zeros(n, 3, dtype=single.dtype)
    else:
        R, t = frames_from_atoms(torch.as_tensor(init_pos).to(single.dtype).detach())
    keys = jax_prng.split(key, depth) if key is not None else [None] * depth
    traj = []
    fp = P.sub("fold_iteration/")
    for i in range(depth):
        act, R, t = fold_iteration(act, R, t, act_2d, mask, fp, keys[i], use_dropout)
        traj.append(torch.cat([R, (POSITION_SCALE * t)[..., None]], -1))
    return act, torch.stack(traj)


# ------------------------------------------------ sidechain, atom14 and heads
# folding_multimer.py:950-1040 (MultiRigidSidechain), all_atom_multimer.py:
# 370-468 (torsion_angles_to_frames, frames_and_literature_positions_to_
# atom14_pos), modules.py:777-1120 (the four heads).  The residue tables are
# inputs (`tables`: default_frame [21,8,4,4], atom14_to_group [21,14],
# atom14_lit_pos [21,14,3], atom14_mask [21,14]), as the reference's native
# structure module reads them from its weights directory (const/...).

def _compose(Ra, ta, Rb, tb):
    """Rigid composition (Ra, ta) @ (Rb, tb) = (Ra Rb, Ra tb + ta)."""
    return Ra @ Rb, (Ra @ tb[..., None])[..., 0] + ta


def torsion_angles_to_frames(aatype, R, t, sin_cos, tables):
    """all_atom_multimer.py:370-435: default frames of the residue type
    composed with a rotation about x by each torsion (backbone group: none),
    chi2..chi4 chained onto the previous chi frame, all mapped by the backbone
    frame (R, t).  Returns the 8 global frames (R [N,8,3,3], t [N,8,3])."""
    dt_ = sin_cos.dtype
    m = torch.as_tensor(np.asarray(tables["default_frame"]), dtype=dt_)[aatype]
    dR, dtr = m[..., :3, :3], m[..., :3, 3]
    n = aatype.shape[0]
    s = torch.cat([torch.zeros(n, 1, dtype=dt_), sin_cos[..., 0]], -1)
    c = torch.cat([torch.ones(n, 1, dtype=dt_), sin_cos[..., 1]], -1)
    z, o = torch.zeros_like(s), torch.ones_like(s)
    rot = torch.stack([o, z, z, z, c, -s, z, s, c], -1).reshape(n, 8, 3, 3)
    fR, ft = dR @ rot, dtr
    cR, ct = [fR[:, g] for g in range(8)], [ft[:, g] for g in range(8)]
    for g in (5, 6, 7):  # chi2..chi4 frames map to the previous chi frame
        cR[g], ct[g] = _compose(cR[g - 1], ct[g - 1], fR[:, g], ft[:, g])
    BR, Bt = torch.stack(cR, 1), torch.stack(ct, 1)
    return _compose(R[:, None], t[:, None], BR, Bt)


def frames_to_atom14(aatype, GR, Gt, tables):
    """all_atom_multimer.py:438-468: each atom's literature position mapped by
    its rigid group's global frame, masked to the atoms the type has."""
    dt_ = GR.dtype
    grp = torch.as_tensor(np.asarray(tables["atom14_to_group"])).long()[aatype]
    oh = torch.nn.functional.one_hot(grp, 8).to(dt_)
    Ra = torch.einsum("nag,ngij->naij", oh, GR)
    ta = torch.einsum("nag,ngi->nai", oh, Gt)
    lit = torch.as_tensor(np.asarray(tables["atom14_lit_pos"]), dtype=dt_)[aatype]
    mask = torch.as_tensor(np.asarray(tables["atom14_mask"]), dtype=dt_)[aatype]
    return ((Ra @ lit[..., None])[..., 0] + ta) * mask[..., None]


def multi_rigid_sidechain(R, t, act, initial_act, aatype, p, tables):
    """folding_multimer.py:950-1040 (num_channel 128, 2 residual blocks):
    input projections of relu(act) and relu(initial_act) (haiku names
    input_projection, input_projection_1), residual blocks (resblock1/2,
    then resblock1_1/2_1), 7 torsions as l2-normalised (sin, cos) pairs
    (eps 1e-12, :927-932), frames, atom14 positions.  (R, t) is the
    backbone frame with its translation in angstroms."""
    relu = torch.relu
    a = linear(relu(act), p.sub("input_projection/")) + \
        linear(relu(initial_act), p.sub("input_projection_1/"))
    for b in range(2):
        sfx = "" if b == 0 else "_1"
        old = a
        a = linear(relu(a), p.sub(f"resblock1{sfx}/"))
        a = linear(relu(a), p.sub(f"resblock2{sfx}/"))
        a = a + old
    un = linear(relu(a), p.sub("unnormalized_angles/")).reshape(-1, 7, 2)
    ang = un / torch.sqrt(torch.clamp((un * un).sum(-1, keepdim=True), min=1e-12))
    GR, Gt = torsion_angles_to_frames(aatype, R, t, ang, tables)
    return frames_to_atom14(aatype, GR, Gt, tables)


def heads(pair, act, single, params, dtype=torch.float64):
    """modules.py:1091-1120 (distogram: half_logits + its transpose over the
    residue axes), :835-873 (predicted aligned error, not symmetrised),
    :777-833 (pLDDT on the structure module's act: LayerNorm, act_0 relu,
    act_1 relu, logits), :875-900 (experimentally resolved on the trunk
    single, 37 logits)."""
    P = Params(params, "param/", dtype)
    h = linear(pair, P.sub("distogram_head/half_logits/"))
    dgram = h + h.transpose(0, 1)
    pae = linear(pair, P.sub("predicted_aligned_error_head/logits/"))
    L = P.sub("predicted_lddt_head/")
    x = layer_norm(act, L("input_layer_norm/scale"), L("input_layer_norm/offset"))
    x = torch.relu(linear(x, L.sub("act_0/")))
    x = torch.relu(linear(x, L.sub("act_1/")))
    plddt = linear(x, L.sub("logits/"))
    expres = linear(single, P.sub("experimentally_resolved_head/logits/"))
    return dgram, pae, plddt, expres


def structure_heads(single, pair, mask, aatype, params, depth, key, use_dropout, tables,
                    dtype=torch.float64, init_pos=None):
    """The post-trunk step of the reference's StructureHeadsFwd
    (native/ffi.cu:530-575): the fold iterations (folding_multimer.py:
    476-548), the last iteration's sidechain on [act, initial_act] with the
    backbone frame scaled to angstroms (:465-466; final_atom14_positions,
    :604-606), and the heads.  Returns (atom14 [N,14,3], distogram [N,N,64],
    pae [N,N,64], plddt [N,50], experimentally resolved [N,37])."""
    act, traj = fold(single, pair, mask, params, depth, key, use_dropout, dtype, init_pos)
    P = Params(params, "param/", dtype)
    init = layer_norm(single, P("single_layer_norm/scale"), P("single_layer_norm/offset"))
    aat = torch.as_tensor(aatype).long().clamp(0, 20)
    atom14 = multi_rigid_sidechain(traj[-1][..., :3], traj[-1][..., 3], act, init, aat,
                                   P.sub("fold_iteration/rigid_sidechain/"), tables)
    return (atom14,) + heads(pair, act, single, params, dtype)


# ------------------------------------------------------------------ recycling
# modules_multimer.py:487-507 (the three prev_* terms of the embedder) and
# bindcraft/af2.py:195-202 (recycled_alphafold_outputs).
PREV_POS_BINS, PREV_POS_MIN, PREV_POS_MAX = 15, 3.25, 20.75  # config.py prev_pos
GLY = 7  # residue_constants.restype_order['G']


def pseudo_beta_atom14(aatype, atom14):
    """pseudo_beta_fn (modules.py:1249-1264, no mask): CB, or CA for glycine,
    read from atom14 positions (CA is slot 1, CB slot 4 of every residue
    type's atom14 list, the same atoms atom37 slots 1 and 3 hold)."""
    gly = torch.as_tensor(np.asarray(aatype)).long() == GLY
    return torch.where(gly[:, None], atom14[:, 1], atom14[:, 4])


def dgram_from_positions(pos, num_bins=PREV_POS_BINS, min_bin=PREV_POS_MIN, max_bin=PREV_POS_MAX):
    """modules.py:1215-1238: one-hot of the squared distance between the
    squared lower breaks linspace(min, max, bins)^2 (strict on both sides;
    the last bin is open to 1e8).  Breaks in float32, as the JAX computes
    them; a zero distance lies in no bin."""
    lower = torch.linspace(min_bin, max_bin, num_bins, dtype=torch.float32).to(pos.dtype) ** 2
    upper = torch.cat([lower[1:], torch.tensor([1e8], dtype=pos.dtype)])
    d2 = ((pos[:, None, :] - pos[None, :, :]) ** 2).sum(-1, keepdim=True)
    return ((d2 > lower) & (d2 < upper)).to(pos.dtype)


def recycle_terms(aatype, prev_atom14, prev_pair, prev_msa0, p_emb, dtype=torch.float64):
    """The embedder's three recycle terms (modules_multimer.py:487-507):
    pair += prev_pos_linear(dgram(pseudo_beta(prev_pos))) +
    prev_pair_norm(prev_pair); msa[0] += prev_msa_first_row_norm(prev_msa0).
    With the previous state all zero (the first pass) they are the Linear's
    bias plus the pair norm's offset, and the msa norm's offset: a
    LayerNorm of a zero vector is its offset, and a zero distance lies in
    no bin.  Returns (pair term [N,N,128], msa row-0 term [N,256])."""
    P = Params(p_emb, "param/", dtype)
    dg = dgram_from_positions(pseudo_beta_atom14(aatype, prev_atom14))
    pair_t = linear(dg, P.sub("prev_pos_linear/")) + layer_norm(
        prev_pair, P("prev_pair_norm/scale"), P("prev_pair_norm/offset"))
    msa_t = layer_norm(prev_msa0, P("prev_msa_first_row_norm/scale"),
                       P("prev_msa_first_row_norm/offset"))
    return pair_t, msa_t


# ------------------------------------------------------------ template row
# modules_multimer.py:1080-1137 template_embedding_1d with
# all_atom_multimer.py:854-941 (get_chi_atom_indices, compute_chi_angles) and
# geometry/vector.py:187-212 (dihedral_angle); bindcraft/af2.py:153-160 builds
# the template arrays from the input atoms.

def dihedral_angle(a, b, c, d):
    """geometry/vector.py:187-212: v1 = a - b, v2 = b - c, v3 = d - c,
    c1 = v1 x v2, c2 = v3 x v2, c3 = c2 x c1, atan2(c3 . v2,
    |v2| (c1 . c2)) with |v2| clipped at 1e-6."""
    v1, v2, v3 = a - b, b - c, d - c
    c1, c2 = torch.linalg.cross(v1, v2), torch.linalg.cross(v3, v2)
    c3 = torch.linalg.cross(c2, c1)
    v2n = torch.sqrt(torch.clamp((v2 * v2).sum(-1), min=1e-12))
    return torch.atan2((c3 * v2).sum(-1), v2n * (c1 * c2).sum(-1))


def template_row(template_aatype, atoms37, mask37, p_emb, tables, dtype=torch.float64):
    """The template's MSA row and its mask: features one_hot(aatype, 22),
    sin(chi) m, cos(chi) m, m for the 4 chi angles (chi atoms by
    tables['chi_atom_indices'][aatype], m = tables['chi_angles_mask'][aatype]
    times all four atoms present; aatype 21 (gap) reads the unknown type's
    row 20, as XLA's clamped gather does), then template_single_embedding,
    relu, template_projection; mask = m of chi 1."""
    aat = torch.as_tensor(np.asarray(template_aatype)).long()
    g = aat.clamp(0, 20)
    idx = torch.as_tensor(tables["chi_atom_indices"]).long()[g]            # [N, 4, 4]
    pos = torch.as_tensor(atoms37, dtype=dtype)
    msk = torch.as_tensor(mask37, dtype=dtype)
    n = pos.shape[0]
    ar = torch.arange(n)[:, None, None]
    pts = pos[ar, idx]                                                      # [N, 4, 4, 3]
    chi = dihedral_angle(pts[..., 0, :], pts[..., 1, :], pts[..., 2, :], pts[..., 3, :])
    m = torch.as_tensor(tables["chi_angles_mask"], dtype=dtype)[g] * msk[ar, idx].prod(-1)
    feat = torch.cat([torch.nn.functional.one_hot(aat, 22).to(dtype), torch.sin(chi) * m,
                      torch.cos(chi) * m, m], -1)
    P = Params(p_emb, "param/", dtype)
    h = torch.relu(linear(feat, P.sub("template_single_embedding/")))
    return linear(h, P.sub("template_projection/")), m[:, 0]


def design_step(target_feat, msa_feat, ids, offset, seq_mask, act_const, aatype, emsa, prm,
                depths, keys, use_dropout, tables, recycles=0, tpl_row=None,
                dtype=torch.float64, init_pos=None, on_pass=None):
    """The trunk of one design step, input features to the structure-module
    outputs (modules_multimer.py:441-700, EmbeddingsAndEvoformer, then
    AlphaFoldIteration's structure module and heads): the embedder plus the
    three recycle terms; the template embedding added to the pair (:530-551,
    act_const = its eight constant projections, None = no template); the
    extra-MSA stack with its mask at zero (the design step's extra MSA;
    `emsa` is any [S_e, N, 64]); the main stack; single =
    single_activations(msa[0]); structure_heads.  `prm` maps 'emb', 'tpl',
    'extra', 'main', 'post' to flat parameter dicts; `depths` and `keys`
    ('tpl', 'extra', 'main', 'fold') give each stack its depth and its JAX
    key.  With `recycles` > 0 the step runs that many forward-only passes
    first (bindcraft/af2.py:195-202), each feeding its atoms, pair and
    msa[0] to the next pass's recycle terms under stop_gradient; `keys` is
    then a list of recycles + 1 such dicts, one per pass.  tpl_row = (row
    [N, 256], mask [N]) is the template's MSA row, appended to the main
    stack's msa and msa mask (modules_multimer.py:608-617).  init_pos
    [N,37,3]: the first pass's structure module starts from these atoms'
    frames, each later pass from the previous pass's atom37 positions
    (native/design_step.cuh:1112-1114, the model's initial_atom_pos).
    on_pass(p, atom14) is called with each forward-only pass's atoms and
    may return the atoms the next pass's recycle terms take instead (a
    test hook: a checker feeds the kernels' own atoms, so a distogram bin
    that rounding moves does not differ between the two)."""
    keys = keys if isinstance(keys, (list, tuple)) else [keys]
    if len(keys) != recycles + 1:
        raise ValueError("design_step: one key dict per pass")
    n = target_feat.shape[0]
    prev = (torch.zeros(n, 14, 3, dtype=dtype), torch.zeros(n, n, 128, dtype=dtype),
            torch.zeros(n, 256, dtype=dtype))
    pmask = seq_mask[:, None] * seq_mask[None, :]
    for p in range(recycles + 1):
        final = p == recycles
        with (torch.enable_grad() if final else torch.no_grad()):
            msa, pair = embedder(target_feat, msa_feat, *ids, prm["emb"], offset=offset,
                                 dtype=dtype)
            pair_t, msa_t = recycle_terms(aatype, *prev, prm["emb"], dtype)
            pair = pair + pair_t
            msa = torch.cat([msa[:1] + msa_t[None], msa[1:]], 0)
            mmask = seq_mask[None].expand(msa.shape[0], -1)
            if tpl_row is not None:
                msa = torch.cat([msa, tpl_row[0][None].to(dtype)], 0)
                mmask = torch.cat([mmask, tpl_row[1][None].to(dtype)], 0)
            k = keys[p]
            if act_const is not None:
                pair = pair + template_embedding(pair, act_const, pmask, prm["tpl"], depths["tpl"],
                                                 k["tpl"], use_dropout, dtype)
            emask = torch.zeros(emsa.shape[:2], dtype=dtype)
            _, pair = evoformer_stack(emsa, pair, emask, pmask, prm["extra"], depths["extra"],
                                      k["extra"], use_dropout, is_extra_msa=True, dtype=dtype)
            msa, pair = evoformer_stack(msa, pair, mmask, pmask, prm["main"], depths["main"],
                                        k["main"], use_dropout, dtype=dtype)
            single = linear(msa[0], Params(prm["emb"], "param/single_activations/", dtype))
            start = None
            if init_pos is not None:
                start = (torch.as_tensor(init_pos) if p == 0 else
                         atom14_to_atom37(prev[0], aatype, seq_mask, tables)[0])
            out = structure_heads(single, pair, seq_mask, aatype, prm["post"], depths["fold"],
                                  k["fold"], use_dropout, tables, dtype, init_pos=start)
        if not final:
            atoms = out[0].detach()
            if on_pass is not None:
                sub = on_pass(p, atoms)
                atoms = atoms if sub is None else torch.as_tensor(sub, dtype=dtype)
            prev = (atoms, pair.detach(), msa[0].detach())
    return out


# ---------------------------------------------------------------------------
# The design sequence's features and the trunk inputs built from them.

OMITTED_AMINO_ACID_LOGIT = -10000.0  # bindcraft/sequence_optimization.py:33


def sequence_features(logits, flags, softmax_weight, one_hot_weight, temperature, logit_scale,
                      bias=None):
    """(features, profile) of the designed logits [N, 20]
    (bindcraft/af2.py:99-104 prepare_design_sequence_features over
    bindcraft/sequence_optimization.py:35-52): p = softmax(logits *
    logit_scale / temperature + bias); f = sw p + (1 - sw) (logits, zero
    where omitted); out = ohw onehot(argmax p) + (1 - ohw) f with the one-hot
    straight-through (stop_gradient(onehot - p) + p); the profile is the same
    with one_hot_weight = 1.  Residues without the DESIGN flag (bit 0) keep
    their logits in both."""
    def feats(ohw):
        scaled = logits * logit_scale / temperature
        p = torch.softmax(scaled if bias is None else scaled + bias, -1)
        blended = torch.where(logits <= OMITTED_AMINO_ACID_LOGIT / 2, torch.zeros_like(logits),
                              logits)
        f = softmax_weight * p + (1 - softmax_weight) * blended
        oh = torch.nn.functional.one_hot(p.argmax(-1), p.shape[-1]).to(p.dtype)
        return ohw * ((oh - p).detach() + p) + (1 - ohw) * f

    designed = torch.as_tensor((np.asarray(flags) & 1) != 0)[:, None]
    return (torch.where(designed, feats(one_hot_weight), logits),
            torch.where(designed, feats(1.0), logits))


def design_inputs(feat, prof):
    """target_feat [N, 21], msa_feat [1, N, 49] and aatype of the sequence
    features (bindcraft/af2.py:187-192: target_feat = the features, msa_feat
    channels 0..19 = features and 25..44 = profile, aatype = argmax; the
    multimer embedder pads target_feat with one zero column,
    modules_multimer.py:450)."""
    n = feat.shape[0]
    tf = torch.cat([feat, torch.zeros(n, 1, dtype=feat.dtype)], -1)
    z = lambda k: torch.zeros(n, k, dtype=feat.dtype)
    mf = torch.cat([feat, z(5), prof, z(4)], -1)[None]
    return tf, mf, feat.detach().argmax(-1).numpy().astype(np.float32)


def atom14_to_atom37(atom14, aatype, seq_mask, tables):
    """all_atom.atom14_to_atom37 as the design step uses it: a gather by
    residx_atom37_to_atom14 times atom37_atom_exists =
    restype_atom37_mask[aatype] * seq_mask (bindcraft/af2.py:187-192 builds
    both from aatype).  tables['atom37_to_atom14'], ['atom37_mask'] [21, 37].
    Returns (atom37 [N, 37, 3], exists [N, 37])."""
    aat = torch.as_tensor(np.asarray(aatype)).long().clamp(0, 20)
    idx = torch.as_tensor(tables["atom37_to_atom14"]).long()[aat]            # [N, 37]
    ex = torch.as_tensor(tables["atom37_mask"], dtype=atom14.dtype)[aat] * seq_mask[:, None]
    a37 = torch.gather(atom14, 1, idx[..., None].expand(-1, -1, 3)) * ex[..., None]
    return a37, ex


def kabsch(coords, ref, weights):
    """bindcraft/protein.py:75-83: weighted centroids, covariance
    ((x - xc) w)^T (y - yc) (the identity when no weight is set), SVD, and the
    rotation R = V diag(1, 1, sign det(V U^T)) U^T that maps centred coords
    onto centred ref.  Returns (R, coords centre, ref centre)."""
    w = weights.to(coords.dtype)
    ws = w.sum() + 1e-8
    xc = (coords * w[:, None]).sum(0) / ws
    yc = (ref * w[:, None]).sum(0) / ws
    cov = ((coords - xc) * w[:, None]).T @ (ref - yc)
    if float(w.sum()) <= 0:
        cov = torch.eye(3, dtype=coords.dtype)
    u, _, vt = torch.linalg.svd(cov)
    d = torch.sign(torch.linalg.det(vt.T @ u.T))
    R = (vt.T * torch.tensor([1.0, 1.0, float(d)], dtype=coords.dtype)) @ u.T
    return R, xc, yc


DESIGN, TEMPLATE, CYCLIC = 1, 2, 64  # bindcraft/protein.py:42-51 ResidueFlags
CA37 = 1                 # residue_constants.atom_order['CA']
CYCLIC_MODES = ("distance", "direction", "neighbours")  # bindcraft/settings.py:87


def cyclic_sequence_offsets(residue_index, asym_id, flags, seq_mask, mode):
    """bindcraft/af2.py:174-185: residue_index differences, except between
    two unmasked CYCLIC residues of one chain, where the ring distance
    min(|d|, L - |d|) (L = the chain's unmasked residue count) takes d's
    sign; 'direction' and 'neighbours' negate it where the short way round
    is the other way, 'neighbours' then saturates beyond 2 at +-32."""
    ri = np.asarray(residue_index, np.int64)
    asym = np.asarray(asym_id)
    sm = np.asarray(seq_mask, np.float64)
    off = ri[:, None] - ri[None, :]
    same = asym[:, None] == asym[None, :]
    clen = (same * sm[None, :]).sum(-1)
    cyc = ((np.asarray(flags).astype(np.int64) & CYCLIC) != 0) * sm
    pairs = same * cyc[:, None] * cyc[None, :]
    dist = np.minimum(np.abs(off), clen[:, None] - np.abs(off))
    if mode in ("direction", "neighbours"):
        dist = np.where(dist < np.abs(off), -dist, dist)
    if mode == "neighbours":
        dist = np.where(np.abs(dist) > 2, 32 * np.sign(dist), dist)
    return np.where(pairs != 0, dist * np.sign(off), off).astype(np.int32)


def flexible_target_residues(residue_index, template_mask, flexibility):
    """bindcraft/af2.py:150-151: every template residue (not designed) whose
    index i has floor((i + 1) f) > floor(i f), in float32 as JAX computes it."""
    i = np.asarray(residue_index, np.float32)
    f = np.float32(flexibility)
    return np.asarray(template_mask, bool) & (np.floor((i + 1) * f) > np.floor(i * f))


def align_to_template(atom37, exists, tpl_atoms37, tpl_mask37, flags):
    """bindcraft/af2.py:89-97 align_prediction_to_target_template: Kabsch of
    the predicted CA (under stop_gradient) onto the template's CA over the
    TEMPLATE-and-not-DESIGN residues whose template CA exists, then every
    predicted atom moved by it; atoms that do not exist are zero."""
    f = np.asarray(flags).astype(np.int64)
    sel = torch.as_tensor(((f & TEMPLATE) != 0) & ((f & DESIGN) == 0))
    w = (sel & (torch.as_tensor(tpl_mask37)[:, CA37] > 0)).to(atom37.dtype)
    R, xc, yc = kabsch(atom37[:, CA37].detach(), torch.as_tensor(tpl_atoms37)[:, CA37].to(
        atom37.dtype), w)
    out = (atom37 - xc) @ R.T + yc
    return out * exists[..., None]


def design_step_seq(logits, flags, scalars, ids, offset, seq_mask, act_const, emsa, prm, depths,
                    keys, use_dropout, tables, bias=None, recycles=0, tpl_atoms37=None,
                    tpl_mask37=None, cyclic_mode=None, flexibility=0.0,
                    initial_atom_pos=False, dtype=torch.float64, on_pass=None):
    """design_step from the designed logits: sequence_features ->
    design_inputs -> design_step (one MSA row).  With template atoms
    (tpl_atoms37 [N,37,3], tpl_mask37 [N,37]) the outputs gain the predicted
    atom37 positions aligned onto the template, and their exists mask (the
    reference step's first two outputs, native/design_step.cuh:77-80); with
    a template embedding (act_const) as well, the template's MSA row joins
    the main stack (modules_multimer.py:608-617, the reference's S = 2).
    cyclic_mode (one of CYCLIC_MODES) replaces `offset` by the cyclic
    sequence offsets (bindcraft/af2.py:193); flexibility > 0 turns the
    flexible target residues into gaps of the template (af2.py:153-157);
    initial_atom_pos starts the structure module from tpl_atoms37 (af2.py:193,
    large_complex_initialization)."""
    feat, prof = sequence_features(logits, flags, *scalars, bias=bias)
    tf, mf, aatype = design_inputs(feat, prof)
    if cyclic_mode is not None:
        offset = torch.as_tensor(cyclic_sequence_offsets(ids[0], ids[1], flags, seq_mask,
                                                         cyclic_mode))
    row = None
    if act_const is not None and tpl_atoms37 is not None:
        # bindcraft/af2.py:153-160: the template covers the TEMPLATE residues,
        # minus the flexible ones (a gap, their side chains unmasked out)
        fl = np.asarray(flags).astype(np.int64)
        tres = (fl & TEMPLATE) != 0
        flex = (flexible_target_residues(ids[0], tres & ((fl & DESIGN) == 0), flexibility)
                if flexibility else np.zeros_like(tres))
        t_aat = np.where(tres & ~flex, np.asarray(aatype), 21)
        t_pos = np.where(tres[:, None, None], np.asarray(tpl_atoms37), 0.0)
        side = np.arange(37) > 4  # everything past N, CA, C, CB, O
        t_msk = np.asarray(tpl_mask37) * tres[:, None] * ~(flex[:, None] & side[None])
        row = template_row(t_aat, t_pos, t_msk, prm["emb"], tables, dtype)
    out = design_step(tf, mf, ids, offset, seq_mask, act_const, aatype, emsa, prm, depths, keys,
                      use_dropout, tables, recycles=recycles, tpl_row=row, dtype=dtype,
                      init_pos=(torch.as_tensor(np.asarray(tpl_atoms37), dtype=dtype)
                                if initial_atom_pos else None), on_pass=on_pass)
    if tpl_atoms37 is None:
        return out
    a37, ex = atom14_to_atom37(out[0], aatype, seq_mask, tables)
    return tuple(out) + (align_to_template(a37, ex, tpl_atoms37, tpl_mask37, flags), ex)


# ---------------------------------------------------------------------------
# Confidence metrics of the head logits.

def _tm_score(pae_logits, breaks, residue_weights, asym=None):
    """AF2's predicted_tm_score with its per-alignment vector
    (bindcraft/af/alphafold/common/confidence.py:113-176): d0 from the
    clipped residue-weight sum, T = E_softmax[1 / (1 + c^2 / d0^2)], per
    alignment the pair-weight-normalised sum, the score the weighted max."""
    step = breaks[1] - breaks[0]
    centres = torch.cat([breaks + step / 2, (breaks[-1:] + 1.5 * step)])
    d0 = 1.24 * (torch.clamp(residue_weights.sum(), min=19) - 15) ** (1.0 / 3) - 1.8
    probs = torch.softmax(pae_logits, -1)
    term = (probs * (1.0 / (1 + centres ** 2 / d0 ** 2))).sum(-1)
    n = residue_weights.shape[0]
    mask = (torch.ones(n, n, dtype=torch.bool) if asym is None
            else torch.as_tensor(asym)[:, None] != torch.as_tensor(asym)[None, :])
    term = term * mask
    w = mask * (residue_weights[None, :] * residue_weights[:, None])
    per = (term * (w / (1e-8 + w.sum(-1, keepdim=True)))).sum(-1)
    return (per * residue_weights).max(), per


def confidence(plddt_logits, pae_logits, expres_logits, seq_mask, interface_asym):
    """alphafold_prediction_metrics (bindcraft/af2.py:197-219): pLDDT from the
    50 lddt bins, the PAE expectation symmetrised, pTM, ipTM and its
    per-residue vector (residue_weights = seq_mask), sigmoid of the CA
    experimentally-resolved logit.  The PAE head's breaks are
    linspace(0, 31, 63)."""
    dt = pae_logits.dtype
    nb = plddt_logits.shape[-1]
    bw = 1.0 / nb
    centres_l = torch.arange(0.5 * bw, 1.0, bw, dtype=dt)[:nb]
    plddt = (torch.softmax(plddt_logits, -1) * centres_l).sum(-1)
    breaks = torch.linspace(0, 31, pae_logits.shape[-1] - 1, dtype=dt)
    step = breaks[1] - breaks[0]
    centres = torch.cat([breaks + step / 2, breaks[-1:] + 1.5 * step])
    pae = (torch.softmax(pae_logits, -1) * centres).sum(-1)
    pae = (pae + pae.T) / 2
    ptm, _ = _tm_score(pae_logits, breaks, seq_mask)
    iptm, iptm_pr = _tm_score(pae_logits, breaks, seq_mask, interface_asym)
    return plddt, pae, ptm.reshape(1), iptm.reshape(1), iptm_pr, torch.sigmoid(expres_logits[:, 1])
