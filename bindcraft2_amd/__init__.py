"""bindcraft2_amd -- MI355X-native AlphaFold2 trunk for BindCraft2.

The product is the C-ABI library ``libbc2n.so`` (declared in
``include/bc2n.h``), built from the HIP sources in ``csrc/`` for gfx950.
This package loads it with ctypes and exposes thin torch-tensor wrappers
(``bindcraft2_amd.ops``) in the shape of the reference's module interface.
There is no CPU fallback: if the library is missing every op raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libbc2n.so")
_lib = None


class NativeError(RuntimeError):
    """A bc2n C-ABI call returned a non-zero status."""


def lib():
    """The loaded libbc2n.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                " (there is no CPU fallback)")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    c = ctypes
    vp, i, f, u32, sz, cs = c.c_void_p, c.c_int, c.c_float, c.c_uint32, c.c_size_t, c.c_char_p
    L.bc2n_last_error.restype = cs
    L.bc2n_abi_version.restype = i
    sigs = {
        "bc2n_triattn_save_bytes": (sz, [i, i, i]),
        "bc2n_triattn_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp]),
        "bc2n_triattn_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_triattn_fwd_noalloc": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp]),
        "bc2n_trimul_save_bytes": (sz, [i, i, i]),
        "bc2n_trimul_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp]),
        "bc2n_trimul_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_transition_save_bytes": (sz, [c.c_long, i, i]),
        "bc2n_transition_fwd": (i, [vp, cs, cs, c.c_long, i, vp, vp, vp, vp]),
        "bc2n_transition_bwd": (i, [vp, cs, cs, c.c_long, i, vp, vp, vp, vp, vp]),
        "bc2n_opm_save_bytes": (sz, [i, i, i, i]),
        "bc2n_opm_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_opm_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp, vp]),
        "bc2n_msarow_save_bytes": (sz, [i, i, i, i]),
        "bc2n_msarow_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_msarow_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp, vp, vp]),
        "bc2n_msacol_save_bytes": (sz, [i, i, i, i]),
        "bc2n_msacol_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp]),
        "bc2n_msacol_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_msaglobal_save_bytes": (sz, [cs, cs, i, i]),
        "bc2n_msaglobal_fwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp]),
        "bc2n_msaglobal_bwd": (i, [vp, cs, cs, i, i, vp, vp, vp, vp, vp, vp]),
        "bc2n_evoformer_save_bytes": (sz, [cs, i, i, c.c_int64, c.c_int64]),
        "bc2n_evoformer_detached_bytes": (sz, [cs, i, i, c.c_int64, c.c_int64]),
        "bc2n_save_slots_probe": (i, [cs, i, i, i, i]),
        "bc2n_set_save_policy": (i, [i]),
        "bc2n_set_msa_overlap": (i, [i]),
        "bc2n_evoformer_replays": (i, [cs, i, i, c.c_int64, c.c_int64]),
        "bc2n_stack_prealloc": (i, [i, i, i, cs, i, i, i]),
        "bc2n_tplstack_prealloc": (i, [i, i, cs]),
        "bc2n_sm_prealloc": (i, [i, i, cs]),
        "bc2n_tplembed_prealloc": (i, [i, i, cs]),
        "bc2n_evoformer_fwd": (i, [vp, vp, vp, vp, vp, vp, i, i, i, i, c.c_int64, c.c_int64,
                                   c.c_int64, c.c_int64, c.c_int64, c.c_int64, cs, vp, vp, vp, vp]),
        "bc2n_evoformer_bwd": (i, [vp, vp, vp, vp, vp, vp, vp, vp, i, i, i, i, c.c_int64,
                                   c.c_int64, c.c_int64, c.c_int64, c.c_int64, cs, vp, vp]),
        "bc2n_tplstack_save_bytes": (sz, [cs, i, c.c_int64]),
        "bc2n_tplstack_fwd": (i, [vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs, vp, vp]),
        "bc2n_tplstack_bwd": (i, [vp, vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs, vp]),
        "bc2n_tplembed_save_bytes": (sz, [cs, i, c.c_int64]),
        "bc2n_tplembed_fwd": (i, [vp, vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs, vp, vp]),
        "bc2n_tplembed_bwd": (i, [vp, vp, vp, vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs, vp]),
        "bc2n_embedder_fwd": (i, [vp, vp, vp, vp, vp, vp, vp, vp, i, i, cs, vp, vp]),
        "bc2n_embedder_bwd": (i, [vp, vp, vp, vp, i, i, cs, vp, vp]),
        "bc2n_fold_save_bytes": (sz, [cs, i, c.c_int64]),
        "bc2n_fold_fwd": (i, [vp, vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs, vp, vp, vp]),
        "bc2n_fold_bwd": (i, [vp, vp, vp, vp, vp, vp, vp, i, c.c_int64, c.c_int64, cs, vp, vp]),
        "bc2n_design_step_save_bytes": (sz, [cs, cs, cs, cs, cs, i, i, c.c_int64, c.c_int64,
                                             c.c_int64, c.c_int64]),
        "bc2n_design_step_fwd": (i, [vp] * 11 + [vp, i, i] + [c.c_int64] * 6 + [cs] * 5
                                 + [vp] * 6),
        "bc2n_design_step_bwd": (i, [vp, vp, vp, vp, c.c_int64] + [vp] * 6 + [i, i]
                                 + [c.c_int64] * 5 + [cs] * 5 + [vp, vp]),
        "bc2n_seqfeat_fwd": (i, [vp, vp, vp, vp, f, f, f, f, f, vp, i, vp, vp]),
        "bc2n_seqfeat_bwd": (i, [vp, vp, vp, vp, vp, vp, f, f, f, f, f, vp, i, vp]),
        "bc2n_design_inputs_fwd": (i, [vp, vp, vp, i, vp, vp, vp]),
        "bc2n_design_inputs_bwd": (i, [vp, vp, vp, i, vp, vp]),
        "bc2n_design_step_seq_save_bytes": (sz, [cs, cs, cs, cs, cs, i, c.c_int64, c.c_int64,
                                                 c.c_int64, c.c_int64]),
        "bc2n_design_step_seq_fwd": (i, [vp, vp, vp, vp, vp, f] + [vp] * 8 + [i, vp]
                                     + [c.c_int64] * 7 + [f] + [cs] * 5 + [vp] * 17),
        "bc2n_design_step_seq_bwd": (i, [vp, vp, vp, vp, vp, f, vp, c.c_int64] + [vp] * 14
                                     + [i, vp] + [c.c_int64] * 5 + [cs] * 5 + [vp]),
        "bc2n_confidence_save_bytes": (sz, [i]),
        "bc2n_confidence_fwd": (i, [vp] * 6 + [i] + [vp] * 7),
        "bc2n_confidence_bwd": (i, [vp] * 13 + [i, vp, vp, vp]),
        "bc2n_structure_heads_save_bytes": (sz, [cs, i, c.c_int64]),
        "bc2n_structure_heads_fwd": (i, [vp, vp, vp, vp, vp, vp, i, i, c.c_int64, c.c_int64, cs,
                                         vp, vp, vp, vp, vp, vp]),
        "bc2n_structure_heads_bwd": (i, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i, c.c_int64,
                                         c.c_int64, cs, vp, vp]),
        "bc2n_dropout_table": (i, [vp, vp, i, i, u32, u32, f]),
        "bc2n_bernoulli_bits": (i, [vp, vp, c.c_long, u32, u32, f]),
        "bc2n_stack_keys": (i, [vp, vp, i, vp]),
        "bc2n_prof_enable": (i, [i]),
        "bc2n_prof_filter": (i, [cs]),
        "bc2n_prof_read": (i, [vp, i, vp, vp, i]),
        "bc2n_probe_gemm": (i, [vp, i, i, i, vp, vp, vp]),
        "bc2n_probe_mfma": (c.c_double, [vp, i, i, i, vp]),
        "bc2n_probe_gemm_f32": (i, [vp, i, i, i, i, vp, c.c_long, c.c_long, c.c_long, vp,
                                    c.c_long, c.c_long, c.c_long, vp, c.c_long, c.c_long,
                                    c.c_long]),
        "bc2n_probe_layernorm": (i, [vp, c.c_long, i, vp, vp, vp, i, vp, vp, vp]),
        "bc2n_probe_recycle": (i, [vp, i, cs, vp, vp, vp, vp, vp, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def check(status):
    """Raise NativeError with the library's message for a non-zero status."""
    if status != 0:
        msg = lib().bc2n_last_error().decode(errors="replace")
        raise NativeError(msg or f"bc2n call failed with status {status}")


def exported_symbols():
    """Names declared in include/bc2n.h (the C ABI)."""
    import re
    hdr = os.path.join(os.path.dirname(_HERE), "include", "bc2n.h")
    with open(hdr) as fh:
        txt = fh.read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)  # declarations only, not comments
    txt = re.sub(r"//[^\n]*", "", txt)
    return sorted(set(re.findall(r"\b(bc2n_[a-z0-9_]+)\s*\(", txt)))


def prof_enable(on=True, only=None):
    """Per-kernel event timing on/off; `only`: time just the launches of that
    timer name."""
    check(lib().bc2n_prof_filter(None if only is None else only.encode()))
    check(lib().bc2n_prof_enable(int(on)))


def prof_read(cap=128, name_len=64):
    """{kernel name: (total ms, launches)} since the last read."""
    names = ctypes.create_string_buffer(cap * name_len)
    ms = (ctypes.c_double * cap)()
    cnt = (ctypes.c_int * cap)()
    n = lib().bc2n_prof_read(names, name_len, ms, cnt, cap)
    if n < 0:
        check(1)
    out = {}
    for i in range(n):
        nm = names.raw[i * name_len:(i + 1) * name_len].split(b"\0", 1)[0].decode()
        out[nm] = (ms[i], cnt[i])
    return out
