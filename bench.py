"""Benchmark of the AF2 trunk hot path on one MI355X.

Default workload (the metric's own config): the
trunk of one design gradient step at L=224 -- forward AND backward of
  * the template pair stack: 2 blocks, c_t=64 (native_tplstack_fwd/bwd),
  * the extra-MSA stack: 4 blocks in the reference's pair-only form
    (extra_msa_mask == 0 in the design step),
  * the main Evoformer stack: 48 blocks, N_seq=1, c_m=256, c_z=128
    (native_evoformer_fwd/bwd),
with dropout on (JAX-exact masks from a stack key), random-init weights
(LeCun normal, AF2 gate init) and N(0,1) synthetic activations resident in
HBM, 10% of residues masked.  The same line also carries `design_step_ms`:
the one-call design step from the designed logits (sequence features,
embedder with its recycle terms, template embedding, the template's MSA row
(S = 2 in the main stack, the reference's design shape), the three stacks,
the 8-iteration structure module, heads, confidence metrics, and the atom37
positions superposed on the template) at the reference's design default of
one recycle: a forward-only pass, then the differentiated pass forward and
backward to d(logits) (`design_recycles`).

`--workload triattn` / `trimul` time BASELINE configs[1] / configs[2]
(one module fwd+bwd, both orientations / directions); `--workload design`
the one-call design step alone; `--workload fold` the structure module's 8
fold iterations; `--n 512` any of them at the large complex's length.

Prints ONE JSON line.  `roofline` is the dominant kernel's achieved rate:
its algorithmic work per launch (kernel_model) over its mean launch time,
HIP events recorded on its own stream around its launches alone in a second
pass of the same K steps (events around every launch slow the step by ~10%),
against the MI355X dense MFMA peak or the HBM peak, whichever its arithmetic
intensity puts it under.  `cpu_baseline` times the oracle (fp32 torch-CPU
restatement of the reference's JAX modules) on this host: one Evoformer block
forward at L=64 and, extrapolated from one block of
each kind, the trunk step.
"""
import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ms per design grad step (48-block trunk fwd+bwd) at L=224; triattn/trimul TFLOP/s"
PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0


# ----------------------------------------------------------- algorithmic work
def triattn_flops(n, c=128, h=4):
    """Algorithmic FLOPs of one triangle-attention module, forward+backward."""
    m = n * n
    return (2 * m * c * 4 * c + 2 * m * c * h + 4 * n ** 3 * c + 2 * m * c * c      # fwd
            + 2 * m * c * c + 10 * n ** 3 * c + 2 * m * 4 * c * c + 2 * m * c * h)  # bwd


def trimul_flops(n, c=128, i=128):
    """Forward: projections (4I+C outputs) + contraction + output; backward:
    output dX, two contractions, projection dX."""
    m = n * n
    fwd = 2 * m * c * (4 * i + c) + 2 * i * n ** 3 + 2 * m * i * c
    bwd = 2 * m * c * i + 4 * i * n ** 3 + 2 * m * (4 * i + c) * c
    return fwd + bwd


# Per-launch algorithmic model of the hot kernels at length n (M = n^2
# tokens): (MFMA FLOPs, HBM bytes).  Timer names without a prefix are the
# pair track's launches (C = c_z = 128, H = 4 heads, I = 128, transition
# factor 4); "tpl."-prefixed ones are the template stack's (C = I = 64,
# H = 4 heads of 16, factor 2).  Bytes count each operand read and each
# result written once (binary16 = 2 B, f32 = 4 B); FLOPs are the products the
# kernel executes (the attention backward's recomputed scores included).  A
# kernel whose FLOP/byte is below the machine balance (RIDGE) is HBM-bound on
# the roofline, above it MFMA-bound.  Names of other widths ("msa.") and
# kernels outside the model give None.
RIDGE = PEAK_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)  # 312.5 FLOP/B


def kernel_model(name, n):
    c, h, f = 128, 4, 4
    if name.startswith("tpl."):
        c, h, f, name = 64, 4, 2, name[4:]
    elif name.startswith("msa."):
        return None
    m = n * n
    gemm = lambda k, cols: 2 * m * k * cols
    model = {
        # q|k|v|g read, o and og written, bias, lse, mask
        "attn_fwd": (4 * n ** 3 * c, m * (8 * c + 4 * c + 4 * h + 4 * h + 4)),
        # q,k,v,dO read, dq written, bias, lse + Dsum, mask
        "attn_bwd_dq": (6 * n ** 3 * c, m * (6 * c + 2 * c + 2 * c + 4 * h + 8 * h + 4)),
        # q,dO,k,v read, dk,dv written, bias, lse + Dsum, mask, d(bias) once
        "attn_bwd_dkv": (8 * n ** 3 * c, m * (8 * c + 4 * c + 4 * h + 8 * h + 4 + 4 * h)),
        # left, right read (binary16); T written (f32)
        "trimul.contract_fwd": (2 * c * n ** 3, m * (4 * c + 4 * c)),
        # dT and one operand read, dL or dR written (binary16)
        "trimul.contract_bwd": (2 * c * n ** 3, m * 6 * c),
        "triattn.gemm_qkvg": (gemm(c, 4 * c), m * (2 * c + 8 * c)),
        # input LayerNorm + bias heads + q|k|v|g projection in one kernel (C = 128):
        # pair read, xn + statistics + bias + qkvg written
        # input LayerNorm + the 4I + C projection columns in one kernel (C = 128)
        "trimul.ln_proj": (gemm(c, 5 * c), m * (4 * c + 2 * c + 8 + 4 + 2 * 2 * c + 2 * c)),
        "triattn.ln_qkvg": (gemm(c, 4 * c), m * (4 * c + 2 * c + 8 + 4 * h + 8 * c)),
        "triattn.gemm_out": (gemm(c, c), m * (2 * c + 4 * c + 4 * c)),
        "triattn.gemm_dout": (gemm(c, c), m * (4 * c + 8 * c + 4 * h)),
        "triattn.gemm_dx": (gemm(4 * c, c), m * (8 * c + 4 * c)),
        "trimul.gemm_proj": (gemm(c, 5 * c), m * (2 * c + 4 * c + 2 * c + 4)),
        "trimul.proj_bwd": (gemm(c, 4 * c), m * (2 * c + 4 * c + 4 + 8 * c)),
        "trimul.gemm_out": (gemm(c, c), m * (2 * c + 2 * c + 4 * c + 2 * c + 4 * c)),
        # centre norm + output projection in one kernel (C = 128): T read (f32),
        # statistics, then the output epilogue's traffic
        "trimul.ln_out": (gemm(c, c), m * (4 * c + 8 + 2 * c + 4 * c + 2 * c + 4 * c)),
        "trimul.gemm_dout": (gemm(c, c), m * (4 * c + 2 * c + 2 * c + 4 * c + 2 * c)),
        # with the centre norm's backward in its epilogue: dout, g_out, o read,
        # d(cat)'s gating columns written, T and the statistics read, dT written
        "trimul.gemm_dout_ln": (gemm(c, c), m * (4 * c + 2 * c + 2 * c + 2 * c + 4 * c + 8 + 2 * c)),
        "trimul.gemm_dx": (gemm(5 * c, c), m * (10 * c + 4 * c)),
        # recompute GEMM + d(cat) + dX GEMM + LayerNorm backward: xn, d(left|right),
        # d(cat)'s gating columns, mask, x, dout read, din written, LN stats
        "trimul.tail_bwd": (gemm(c, 4 * c) + gemm(5 * c, c),
                            m * (2 * c + 4 * c + 2 * c + 4 + 4 * c + 4 * c + 4 * c + 8)),
        "trimul.gemm_dx_ln": (gemm(5 * c, c), m * (10 * c + 12 * c + 8)),
        "triattn.gemm_dx_ln": (gemm(4 * c, c), m * (8 * c + 12 * c + 4 * h + 8)),
        "trans.gemm_dx_ln": (gemm(f * c, c), m * (2 * f * c + 12 * c + 8)),
        # the pair transition as one kernel a direction (C = 128): x read, out
        # written, LN statistics, the hidden's mask bits; the hidden stays on chip
        "trans.fused_fwd": (gemm(c, f * c) + gemm(f * c, c), m * (4 * c + 4 * c + 8 + f * c // 8)),
        "trans.fused_bwd": (gemm(c, f * c) + gemm(f * c, c),
                            m * (4 * c + 4 * c + 4 * c + 8 + f * c // 8)),
        "trans.gemm1": (gemm(c, f * c), m * (2 * c + 2 * f * c + f * c // 8)),
        "trans.gemm2": (gemm(f * c, c), m * (2 * f * c + 4 * c + 4 * c)),
        "trans.gemm_dh": (gemm(c, f * c), m * (4 * c + 2 * f * c + f * c // 8)),
        "trans.gemm_dx": (gemm(f * c, c), m * (2 * f * c + 4 * c)),
        "triattn.ln_fwd": (0, m * (6 * c + 4 * h + 8)),
        "triattn.ln_bwd": (0, m * (16 * c + 4 * h + 8)),
        "trimul.ln_fwd": (0, m * (6 * c + 8)),
        "trimul.ln_bwd": (0, m * (16 * c + 8)),
        "trimul.ln_center": (0, m * (6 * c + 8)),
        "trimul.ln_center_bwd": (0, m * (10 * c + 8)),
    }
    return model.get(name)


def kernel_work(name, n):
    """Executed MFMA FLOPs per launch (None for kernels outside the model)."""
    km = kernel_model(name, n)
    return None if km is None else km[0]


# --------------------------------------------------------------- CPU baseline
def cpu_trunk_baseline(n, budget_s=20.0):
    """fp32 torch-CPU oracle: one Evoformer block, one pair-only block and one
    template block forward+backward at length n, scaled to 48 + 4 + 2 blocks."""
    import numpy as np
    import torch
    from bindcraft2_amd import params as bparams
    from oracle import af2, jax_prng

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    f32 = torch.float32
    prm = bparams.init_block_params(0, rng, gates="zero")
    tprm = bparams.init_template_block_params(0, rng, gates="zero")
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    pmask = torch.as_tensor(np.outer(m1, m1))
    mmask = torch.as_tensor(m1[None])
    key = jax_prng.prng_key(1)

    def evo_block():
        pair = torch.randn(n, n, 128, requires_grad=True)
        msa = torch.randn(1, n, 256, requires_grad=True)
        mo, po = af2.evoformer_iteration(msa, pair, mmask, pmask, prm, "param/block0/", key, True,
                                         dtype=f32)
        torch.autograd.grad((po, mo), (pair, msa), (torch.randn_like(po), torch.randn_like(mo)))

    def pair_only_block():
        # the pair track of an Evoformer block (OPM constant + 5 pair modules)
        pair = torch.randn(n, n, 128, requires_grad=True)
        P = af2.Params(prm, "param/block0/", f32)
        x = pair + P("outer_product_mean/output_b") / 1e-3
        for name, fn in (("triangle_multiplication_outgoing", lambda a, p: af2.triangle_multiplication(a, pmask, p, True)),
                         ("triangle_multiplication_incoming", lambda a, p: af2.triangle_multiplication(a, pmask, p, False)),
                         ("triangle_attention_starting_node", lambda a, p: af2.triangle_attention(a, pmask, p, False)),
                         ("triangle_attention_ending_node", lambda a, p: af2.triangle_attention(a, pmask, p, True)),
                         ("pair_transition", lambda a, p: af2.transition(a, pmask, p))):
            x = x + fn(x, P.sub(name + "/"))
        torch.autograd.grad(x, pair, torch.randn_like(x))

    def tpl_block():
        pair = torch.randn(n, n, 64, requires_grad=True)
        out = af2.template_iteration(pair, pmask, tprm, "param/block0/", key, True, dtype=f32)
        torch.autograd.grad(out, pair, torch.randn_like(out))

    def config1_block():
        # one Evoformer block forward at L=64, S=1, fp32,
        # N(0,1) activations, all-ones masks, AF2 gate init, no dropout
        n1 = 64
        with torch.no_grad():
            af2.evoformer_iteration(torch.randn(1, n1, 256), torch.randn(n1, n1, 128),
                                    torch.ones(1, n1), torch.ones(n1, n1), prm, "param/block0/",
                                    None, False, dtype=f32)

    config1_block()  # first-call setup out of the timing
    reps, t0 = 0, time.perf_counter()
    while reps < 50 and time.perf_counter() - t0 < 3.0:
        config1_block()
        reps += 1
    config1_ms = (time.perf_counter() - t0) / reps * 1e3

    times = {}
    spent = 0.0
    for name, fn in (("evo", evo_block), ("pair_only", pair_only_block), ("tpl", tpl_block)):
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el > budget_s / 3 or reps >= 3:
                break
        times[name] = el / reps
        spent += el
    step_ms = (48 * times["evo"] + 4 * times["pair_only"] + 2 * times["tpl"]) * 1e3
    return {"value": round(step_ms, 1), "unit": "ms", "cores": threads, "kind": "port",
            "cpu": cpu_model(), "config1_block_fwd_ms": round(config1_ms, 2),
            "sample": (f"oracle fp32 torch-CPU, one block each fwd+bwd at L={n}: Evoformer "
                       f"{times['evo']:.2f} s, pair-only {times['pair_only']:.2f} s, template "
                       f"{times['tpl']:.2f} s ({spent:.1f} s of CPU work on {threads} threads); "
                       f"step = 48 x Evoformer + 4 x pair-only + 2 x template (extrapolated); "
                       f"config1_block_fwd_ms = one Evoformer block forward at L=64 "
                       f"(BASELINE configs[0]), {reps} reps")}


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_triattn_baseline(n, seconds=12.0):
    import numpy as np
    import torch
    from bindcraft2_amd import params as bparams
    from oracle import af2

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    name = "triangle_attention_starting_node"
    prm = bparams.init_block_params(0, rng, modules=[name], gates="zero")
    P = af2.Params(prm, f"param/block0/{name}/", torch.float32)
    pair = torch.tensor(rng.standard_normal((n, n, 128)), dtype=torch.float32, requires_grad=True)
    m = np.ones(n, np.float32)
    m[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    mask = torch.as_tensor(np.outer(m, m))
    dout = torch.randn(n, n, 128)
    reps, t0 = 0, time.perf_counter()
    while True:
        out = af2.triangle_attention(pair, mask, P, False)
        torch.autograd.grad(out, pair, dout)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 50:
            break
    return {"value": round(triattn_flops(n) * reps / el / 1e12, 4), "unit": "TFLOP/s",
            "cores": threads, "kind": "port", "cpu": cpu_model(),
            "sample": f"oracle fp32 torch-CPU triangle attention (starting node) fwd+bwd at "
                      f"L={n}, {reps} reps in {el:.1f} s on {threads} host threads"}


# ------------------------------------------------------------------- roofline
def traffic_summary(n):
    """The committed counter summary of the trunk step at length n."""
    return os.path.join(ROOT, "profiles", f"traffic_trunk_L{n}.json")


def traffic_of(kernel, n):
    """HBM bytes per launch of `kernel` (per-launch kernel name as the event
    timer records it) from the committed counter summary of the trunk step
    (rocprofv3 FETCH_SIZE / WRITE_SIZE, scaled by a plain copy's reading);
    None if there is no summary for this length."""
    if not os.path.exists(traffic_summary(n)):
        return None
    with open(traffic_summary(n)) as fh:
        summ = json.load(fh)
    if summ.get("L") != n:
        return None
    # the triangle-attention launches are the head-width-32 instantiation (the
    # row-chunk forms for N <= 256); other timer names map to no one symbol
    nb = n // 32
    syms = {"attn_fwd": [f"attn_fwd_rows<32, {nb}>", f"attn_fwd<32, {nb}, 8>"],
            "attn_bwd_dq": [f"attn_bwd_dq_rows<32, {nb}>", f"attn_bwd_dq<32, {nb}, 8>"],
            "attn_bwd_dkv": [f"attn_bwd_dkv_lds<{nb}>", f"attn_bwd_dkv_lds8<{nb}>",
                             f"attn_bwd_dkv<32, {nb}, {8 if nb > 8 else 4}, "
                             f"{8 if nb > 24 else 4 if nb > 8 else 2}>"],
            "trimul.tail_bwd": ["trimul_tail", "_ZN4bc2n12_GLOBAL__N_118trimul_tail_kernelENS0_8TailArgsE"]}.get(kernel, [kernel])
    for sym in syms:
        k = summ["kernels"].get(sym)
        if k is not None:
            return int(k["fetch_bytes"] + k["write_bytes"])
    # GEMM-based timers: the kernel symbol names the epilogue (demangled or
    # mangled); the contraction's output type tells forward from backward
    pat = {"trimul.proj_bwd": r"EpiTrimulProjBwd",
           "trimul.gemm_proj": r"gemm.*EpiTrimulProj(?!Bwd)",
           "trimul.ln_proj": r"^kernel<0, true, EpiTrimulProj\b|lnproj.*EpiTrimulProj",
           "triattn.ln_qkvg": r"^kernel<4, false, EpiScaledCols\b|lnproj.*EpiScaledCols",
           "trans.fused_fwd": r"^fused<.*EpiResidualRows|fused_kernel.*EpiResidualRows",
           "trans.fused_bwd": r"^fused<.*EpiLnBwd|fused_kernel.*EpiLnBwd",
           "trimul.gemm_out": r"EpiTrimulOut",
           "trimul.ln_out": r"EpiTrimulOut",
           "triattn.gemm_dx_ln": r"EpiLnBwd<4>|EpiLnBwdILi4E",
           "trimul.contract_fwd": rf"contract(_kernel)?(<{nb}, .*float>|ILi{nb}E.*fEE)",
           "trimul.contract_bwd": rf"contract(_kernel)?(<{nb}, .*_Float16>|ILi{nb}E.*DF16_EE)"}.get(kernel)
    if pat is None:
        return None
    import re
    hits = [v for k, v in summ["kernels"].items() if re.search(pat, k)]
    if not hits:
        return None
    k = max(hits, key=lambda v: v["calls"])
    return int(k["fetch_bytes"] + k["write_bytes"])


def event_overhead_us(reps=200):
    """Median elapsed time of an empty event pair (two events recorded back
    to back on the idle stream): what bracketing a launch with events adds to
    its measured duration."""
    import torch
    torch.cuda.synchronize()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(reps)]
    for a, b in pairs:
        a.record()
        b.record()
    torch.cuda.synchronize()
    v = sorted(a.elapsed_time(b) for a, b in pairs)
    return v[len(v) // 2] * 1e3


EVENT_OVERHEAD_US = 0.0  # set by main() once the GPU is up


def _rate(name, n, tot_ms, cnt):
    flops, nbytes = kernel_model(name, n)
    us = max(tot_ms / cnt * 1e3 - EVENT_OVERHEAD_US, 1e-3)
    tf = flops / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    bound = "mfma" if flops / nbytes >= RIDGE else "hbm"
    return us, tf, gbs, bound


def roofline_from(prof, n, dom_prof=None):
    """The dominant modelled kernel (largest total time in `prof`): its
    achieved rate in the unit of the bound its arithmetic intensity puts it
    under, timed from `dom_prof` (a pass timing that kernel alone) when
    given."""
    dom = dominant(prof, n)
    if dom is None:
        return None
    tot, cnt = (dom_prof or prof)[dom]
    us, tf, gbs, bound = _rate(dom, n, tot, cnt)
    flops, nbytes = kernel_model(dom, n)
    if bound == "mfma":
        ach, peak, unit = tf, PEAK_MFMA_TFLOPS, "TFLOP/s"
    else:
        ach, peak, unit = gbs, PEAK_HBM_GBS, "GB/s"
    return {"kernel": dom, "bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 4), "traffic": traffic_of(dom, n), "launch_us": round(us, 2),
            "algorithmic_bytes": nbytes, "algorithmic_flops": flops,
            "flop_per_byte": round(flops / nbytes, 1), "ridge": round(RIDGE, 1),
            "mfma_tflops": round(tf, 2), "mfma_frac": round(tf / PEAK_MFMA_TFLOPS, 4),
            "timing": ("events around this kernel's launches alone" if dom_prof else
                       "events around every launch") +
                      f", less the {EVENT_OVERHEAD_US:.2f} us an empty event pair measures",
            "launch_us_events": round(tot / cnt * 1e3, 2)}


def kernel_rooflines(prof, n):
    """Every modelled kernel: MFMA TFLOP/s and HBM GB/s, each as a fraction of
    its peak, and which one bounds it (by arithmetic intensity)."""
    rows = []
    for k, (tot, cnt) in sorted(prof.items(), key=lambda kv: -kv[1][0]):
        if kernel_model(k, n) is None:
            continue
        us, tf, gbs, bound = _rate(k, n, tot, cnt)
        row = {"kernel": k, "us": round(us, 2), "bound": bound, "tflops": round(tf, 1),
               "mfma_frac": round(tf / PEAK_MFMA_TFLOPS, 4), "gbs": round(gbs, 0),
               "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
        if row["mfma_frac"] > 1.0 or row["hbm_frac"] > 1.0:
            # a rate above peak is a byte/FLOP model error, never a result
            row["model_error"] = True
            print(f"bench.py: kernel_model overstates {k} ({row})", file=sys.stderr)
        rows.append(row)
    return rows


def _short_kernel_name(sym):
    """'void bc2n::attn_bwd_dkv_kernel<32, 7>(bc2n::AttnBwdArgs)' ->
    'attn_bwd_dkv<32, 7>' (the event timer's name plus the template
    arguments, which tell head widths and lengths apart)."""
    s = sym.replace("(anonymous namespace)::", "").replace("void ", "").replace("bc2n::", "")
    s = s.split("(")[0] if not s.startswith("_Z") else s
    base, _, targs = s.partition("<")
    base = base.split("::")[-1]
    base = base[:-len("_kernel")] if base.endswith("_kernel") else base
    # template arguments kept whole: they tell lengths, head widths and the
    # GEMM epilogues apart
    return f"{base}<{targs}" if targs else base


def pmc_summarize(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, n, out):
    """Per-kernel HBM bytes per launch from two rocprofv3 --pmc runs of the
    trunk step (FETCH_SIZE, WRITE_SIZE in KiB per dispatch) and the same two
    counters over a device copy of a known size (bench.py --workload copy),
    whose reading fixes each counter's scale."""
    import csv
    import collections

    def per_kernel(path):
        # one entry per kernel name: its largest launch shape (grid size),
        # e.g. the triangle-attention launches of a kernel MSA attention
        # also uses with a smaller grid
        d = collections.defaultdict(lambda: collections.defaultdict(lambda: [0.0, 0, 0]))
        for r in csv.DictReader(open(path)):
            k = _short_kernel_name(r["Kernel_Name"])
            e = d[k][int(r["Grid_Size"])]
            e[0] += float(r["Counter_Value"]) * 1024.0
            e[1] += 1
            e[2] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        return {k: v[max(v)] + [max(v)] for k, v in d.items()}

    def copy_scale(path):
        big = [float(r["Counter_Value"]) * 1024.0 for r in csv.DictReader(open(path))
               if "copyBuffer" in r["Kernel_Name"]]
        return (256 << 20) / max(big)  # the copy moves 256 MiB each way

    fs, ws = copy_scale(copy_fetch_csv), copy_scale(copy_write_csv)
    f, w = per_kernel(fetch_csv), per_kernel(write_csv)
    kern = {}
    for k in f:
        if k not in w:
            continue
        calls = f[k][1]
        kern[k] = {"calls": calls, "grid": f[k][3], "fetch_bytes": round(f[k][0] / calls * fs),
                   "write_bytes": round(w[k][0] / w[k][1] * ws),
                   "us_under_counters": round((f[k][2] + w[k][2]) / (calls + w[k][1]) / 1e3, 2)}
    summ = {"L": n, "copy_scale": {"FETCH_SIZE": round(fs, 4), "WRITE_SIZE": round(ws, 4)},
            "kernels": dict(sorted(kern.items(), key=lambda kv: -kv[1]["fetch_bytes"]))}
    with open(out, "w") as fh:
        json.dump(summ, fh, indent=1)
    return summ


SQ_COUNTERS = ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS",
               "SQ_LDS_BANK_CONFLICT", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES",
               "GRBM_GUI_ACTIVE")


def pmc_sq_summarize(trunk_csv, probe_csv, n, out_json, out_md, top=12):
    """Per-kernel instruction mix and MFMA busy fraction from one rocprofv3
    --pmc pass of SQ_COUNTERS over a trunk step, with the MFMA issue-rate
    probe (bench.py --workload mfma) read by the same counters as the scale:
    a kernel's MFMA busy fraction is its SQ_VALU_MFMA_BUSY_CYCLES per
    GRBM_GUI_ACTIVE cycle divided by the probe's (whose matrix cores are busy
    every cycle).  Counts are per launch, for each kernel's largest launch
    shape."""
    import csv
    import collections

    def per_dispatch(path):
        d = collections.defaultdict(dict)
        for r in csv.DictReader(open(path)):
            key = (r.get("Dispatch_Id") or r.get("Correlation_Id") or r["Kernel_Name"] + r["Start_Timestamp"])
            e = d[key]
            e["name"] = _short_kernel_name(r["Kernel_Name"])
            e["grid"] = int(r["Grid_Size"])
            e["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        return list(d.values())

    probe = [e for e in per_dispatch(probe_csv) if e["name"].startswith("mfma_rate<0")]
    if not probe:
        raise SystemExit("pmc_sq_summarize: no mfma_rate<0> dispatch in the probe csv")
    busy_scale = max(e["SQ_VALU_MFMA_BUSY_CYCLES"] / e["GRBM_GUI_ACTIVE"] for e in probe)
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for e in per_dispatch(trunk_csv):
        if all(c in e for c in SQ_COUNTERS):
            agg[e["name"]][e["grid"]].append(e)
    rows = {}
    for name, shapes in agg.items():
        grid = max(shapes)
        es = shapes[grid]
        mean = {c: sum(x[c] for x in es) / len(es) for c in SQ_COUNTERS}
        us = sum(x["ns"] for x in es) / len(es) / 1e3
        mf = mean["SQ_INSTS_MFMA"]
        rows[name] = {"grid": grid, "launches": len(es), "us": round(us, 2),
                      **{c: round(mean[c]) for c in SQ_COUNTERS},
                      "valu_per_mfma": round(mean["SQ_INSTS_VALU"] / mf, 2) if mf else "-",
                      "salu_per_mfma": round(mean["SQ_INSTS_SALU"] / mf, 2) if mf else "-",
                      "mfma_busy": round(mean["SQ_VALU_MFMA_BUSY_CYCLES"] / mean["GRBM_GUI_ACTIVE"]
                                         / busy_scale, 4),
                      # SQ_INSTS_VALU counts the MFMAs too; a wave64 VALU
                      # instruction holds its SIMD 4 cycles; GRBM_GUI_ACTIVE
                      # sums the 8 XCDs' cycles; 1024 SIMDs
                      "valu_busy": round((mean["SQ_INSTS_VALU"] - mean["SQ_INSTS_MFMA"]) * 4.0
                                         / (1024.0 * mean["GRBM_GUI_ACTIVE"] / 8.0), 4),
                      "total_us": us * len(es)}
    order = sorted(rows, key=lambda k: -rows[k]["total_us"])
    summ = {"L": n, "counters": list(SQ_COUNTERS), "probe_busy_per_cycle": busy_scale,
            "kernels": {k: rows[k] for k in order}}
    with open(out_json, "w") as fh:
        json.dump(summ, fh, indent=1)
    with open(out_md, "w") as fh:
        fh.write(f"| kernel (largest launch, L={n}) | us | VALU | SALU | MFMA | LDS | LDS bank "
                 "conflict cycles | VALU/MFMA | SALU/MFMA | MFMA busy | VALU busy |\n"
                 "|---|---|---|---|---|---|---|---|---|---|---|\n")
        for k in order[:top]:
            r = rows[k]
            fh.write(f"| `{k}` | {r['us']} | {r['SQ_INSTS_VALU']} | {r['SQ_INSTS_SALU']} | "
                     f"{r['SQ_INSTS_MFMA']} | {r['SQ_INSTS_LDS']} | {r['SQ_LDS_BANK_CONFLICT']} | "
                     f"{r['valu_per_mfma']} | {r['salu_per_mfma']} | {r['mfma_busy']} | "
                     f"{r['valu_busy']} |\n")
    return summ


def kernel_table(prof):
    return {k: {"ms_total": round(t, 3), "launches": c, "us_mean": round(t / c * 1e3, 2)}
            for k, (t, c) in sorted(prof.items(), key=lambda kv: -kv[1][0])}


PROGRESS = False  # --progress: a line on stderr per finished step


def _progress(what):
    if PROGRESS:
        import torch
        torch.cuda.synchronize()
        print(f"bench: {what} done", file=sys.stderr, flush=True)


def profiled(step, steps, skip, only=None):
    """A pass of `steps` steps with the per-kernel event timer on (around the
    launches named `only` alone, if given): {name: (total ms, launches)}; {}
    when skipped (--no-kprof).  The pass runs the stacks on one stream (the
    MSA overlap off), so every kernel's time is its own, not shared with a
    kernel of the other stream; the timed steps keep the overlap."""
    if skip:
        return {}
    import bindcraft2_amd as b
    old = b.lib().bc2n_set_msa_overlap(0)
    b.prof_enable(True, only=only)
    try:
        for i in range(steps):
            step()
            _progress(f"profiled step {i}" + (f" ({only})" if only else ""))
        prof = b.prof_read()
    finally:
        b.prof_enable(False)
        b.lib().bc2n_set_msa_overlap(old)
    return prof


def dominant(prof, n):
    """The modelled kernel with the largest total time in `prof`."""
    cand = {k: v for k, v in prof.items() if kernel_model(k, n) is not None}
    return max(cand, key=lambda k: cand[k][0]) if cand else None


def timed(step, steps, warmup):
    import torch
    for i in range(warmup):
        step()
        _progress(f"warmup step {i}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    _progress(f"{steps} timed steps")
    return ms


DESIGN_RECYCLES = 1


def design_step_setup(n, rng, dev, m1):
    """The one-call design step from the designed logits (sequence features,
    embedder, template embedding (2 blocks), extra stack (4, pair only), main
    stack (48), structure module (8 iterations), heads and the confidence
    metrics), forward + backward to the logits, on random weights and inputs:
    returns (step closure, save-set bytes)."""
    import torch
    from bindcraft2_amd import ops, params as bparams, weights as W
    tree = W.init_af2_params(rng, num_blocks=48, extra_blocks=4, template_blocks=2)
    root = tempfile.mkdtemp(prefix="bc2n_bench_ds_")
    tables = bparams.init_residue_tables(rng)
    dirs = [W.embed_weights_from_params(tree, os.path.join(root, "emb")),
            W.tplembed_weights_from_params(tree, os.path.join(root, "tpl")),
            W.stack_weights_from_params(tree, os.path.join(root, "extra"), prefix=W.EXTRA),
            W.stack_weights_from_params(tree, os.path.join(root, "main"), prefix=W.MAIN),
            W.post_weights_from_params(tree, os.path.join(root, "post"), tables=tables)]
    step_mod = ops.DesignStepSeq(*dirs, depths=(2, 4, 48, 8))
    nt = n - 64  # the target; the last 64 residues are designed
    logits = 0.5 * torch.randn(n, 20, device=dev)
    flags = torch.zeros(n, dtype=torch.uint8, device=dev)
    flags[nt:] = 1  # the binder is designed; the target passes through
    flags[:nt] = 2  # the target is the template: its MSA row joins the stack (S = 2)
    logits[:nt] = torch.nn.functional.one_hot(torch.randint(0, 20, (nt,), device=dev), 20).float()
    scalars = torch.tensor([1.0, 0.0, 1.0, 1.0], device=dev)  # the soft stage
    ids = [torch.arange(n, dtype=torch.float32, device=dev),
           (torch.arange(n, device=dev) >= nt).float() + 1,
           (torch.arange(n, device=dev) >= nt).float() + 1, torch.ones(n, device=dev)]
    iasym = (torch.arange(n, device=dev) >= nt).int()
    seqm = torch.as_tensor(m1, device=dev)
    act_const = 0.1 * torch.randn(n, n, 64, device=dev)
    tpl37 = 8.0 * torch.randn(n, 37, 3, device=dev)  # the template's (the input) atoms
    tplm37 = torch.ones(n, 37, device=dev)
    # the reference's design default: one forward-only recycle pass ahead of
    # the differentiated one (settings/core/default.json:38), each pass
    # with its own four stack keys
    seeds = torch.tensor([[0, 11 + i, 1] for i in range(4 * (DESIGN_RECYCLES + 1))],
                         dtype=torch.int64).to(torch.uint32).to(dev)
    save = torch.empty(step_mod.save_bytes(n), dtype=torch.uint8, device=dev)
    cts = [torch.randn(*sh, device=dev) for sh in ((n, 14, 3), (n, n, 64), (n, n, 64),
                                                  (n, 50), (n, 37))]
    conf_cts = [torch.randn(*sh, device=dev) for sh in ((n,), (n, n), (1,), (1,), (n,), (n,))]
    ct37 = torch.randn(n, 37, 3, device=dev)

    def step():
        step_mod.forward(logits, flags, scalars, ids, seqm, act_const=act_const, seeds=seeds,
                         save=save, interface_asym=iasym, recycles=DESIGN_RECYCLES, atom37=True,
                         tpl_atoms37=tpl37, tpl_mask37=tplm37)
        step_mod.backward(cts, logits, flags, scalars, seqm, save, interface_asym=iasym,
                          conf_cts=conf_cts, d_atom37=ct37)

    return step, save.numel()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=224)
    ap.add_argument("--workload", choices=["trunk", "design", "triattn", "trimul", "fold", "copy",
                                           "mfma"],
                    default="trunk")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-summarize", nargs=5, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                                                         "COPY_WRITE_CSV", "OUT_JSON"),
                    help="write the per-kernel HBM traffic summary from rocprofv3 --pmc runs")
    ap.add_argument("--pmc-sq-summarize", nargs=4, metavar=("TRUNK_CSV", "PROBE_CSV", "OUT_JSON",
                                                           "OUT_MD"),
                    help="write the per-kernel instruction mix / MFMA busy table from rocprofv3 "
                         "--pmc runs of the SQ counters")
    ap.add_argument("--no-kprof", action="store_true",
                    help="skip the per-kernel event-timer pass (roofline / kernel table)")
    ap.add_argument("--no-design", action="store_true",
                    help="trunk workload: skip the secondary one-call design-step timing")
    ap.add_argument("--no-msa-overlap", action="store_true",
                    help="run the Evoformer blocks' MSA side on the caller's stream (A/B of the "
                         "default two-stream order)")
    ap.add_argument("--progress", action="store_true",
                    help="print a line on stderr after every step (long profiler runs)")
    args = ap.parse_args()
    global PROGRESS
    PROGRESS = args.progress
    if args.pmc_summarize:
        summ = pmc_summarize(*args.pmc_summarize[:4], args.n, args.pmc_summarize[4])
        print(json.dumps({"kernels": len(summ["kernels"]), "copy_scale": summ["copy_scale"]}))
        return
    if args.pmc_sq_summarize:
        summ = pmc_sq_summarize(*args.pmc_sq_summarize[:2], args.n, *args.pmc_sq_summarize[2:])
        print(json.dumps({"kernels": len(summ["kernels"]),
                          "probe_busy_per_cycle": summ["probe_busy_per_cycle"]}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the trunk runs on one MI355X; "
              "multi-GPU sharding is a design note, not built)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import bindcraft2_amd as b
    from bindcraft2_amd import ops, params as bparams

    dev = torch.device("cuda:0")
    if args.no_msa_overlap:
        b.lib().bc2n_set_msa_overlap(0)
    n = args.n
    rng = np.random.default_rng(0)
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    pmask = torch.as_tensor(np.outer(m1, m1), device=dev)
    mmask = torch.as_tensor(m1[None], device=dev)

    if args.workload == "copy":
        # calibration for the HBM byte counters: one device-to-device copy of
        # a known size per step (FETCH_SIZE / WRITE_SIZE of this kernel,
        # divided by 256 MiB, is the counters' scale factor)
        nbytes = 256 << 20
        src = torch.randn(nbytes // 4, device=dev)
        dst = torch.empty_like(src)
        ms = timed(lambda: dst.copy_(src), args.steps, args.warmup)
        out = {"metric": "device copy bandwidth (read+write)", "value":
               round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
               "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
               "higher_is_better": True, "config": {"workload": "copy", "bytes": nbytes}}
        print(json.dumps(out))
        return
    if args.workload == "mfma":
        # the matrix-core ceiling: the MFMA forms the kernels use, issued from
        # registers by 8 waves a CU (8 independent chains each), and the
        # product's own GEMM kernel on a compute-bound shape
        blocks, iters = 8 * torch.cuda.get_device_properties(dev).multi_processor_count, 256
        rates = {}
        for form, name in ((0, "v_mfma_f32_16x16x32_f16"), (1, "v_mfma_f32_16x16x16_f16"),
                           (2, "v_mfma_f32_32x32x16_f16"), (3, "v_mfma_f32_16x16x32_bf16")):
            box = {}

            def step(form=form):
                box["flops"], _ = ops.probe_mfma(form, blocks, iters, dev)

            ms = timed(step, args.steps, args.warmup)
            rates[name] = round(box["flops"] / (ms * 1e-3) / 1e12, 1)
        g = 8192
        A = torch.randn(g, g, device=dev).half()
        B = torch.randn(g, g, device=dev).half()
        ms = timed(lambda: ops.probe_gemm(A, B), args.steps, args.warmup)
        out = {"metric": "MFMA rate (dense f16, TFLOP/s)", "value": rates["v_mfma_f32_16x16x32_f16"],
               "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "higher_is_better": True, "dtype": "f16", "data": "synthetic",
               "config": {"workload": "mfma issue-rate probe (registers only) and gemm_kernel "
                                      "at M=N=K=8192 (f16 in, f32 out)", "blocks": blocks,
                          "iters": iters},
               "mfma_forms": rates, "peak_published": 2500.0,
               "gemm_8192_tflops": round(2 * g ** 3 / (ms * 1e-3) / 1e12, 1),
               "gemm_8192_ms": round(ms, 3)}
        print(json.dumps(out))
        return
    global EVENT_OVERHEAD_US
    EVENT_OVERHEAD_US = event_overhead_us()
    dom_prof = None  # the roofline kernel's own timing pass
    if args.workload == "fold":
        # BASELINE configs[4]'s structure-module part: 8 fold iterations (IPA,
        # transition, rigid update) forward+backward, f32, dropout on
        depth = 8
        prm = bparams.init_fold_params(rng, final="random")
        wdir = bparams.write_manifest(tempfile.mkdtemp(prefix="bc2n_bench_fold_"), prm)
        fold = ops.Fold(wdir, depth)
        single = torch.randn(n, 384, device=dev)
        pair = torch.randn(n, n, 128, device=dev)
        seqm = torch.as_tensor(m1, device=dev)
        seed = ops.seed_tensor((0, 7), True, dev)
        d_act = torch.randn(n, 384, device=dev)
        d_traj = torch.randn(depth, n, 3, 4, device=dev)
        save = torch.empty(fold.save_bytes(n), dtype=torch.uint8, device=dev)

        def step():
            fold.forward(single, pair, seqm, seed, save=save)
            fold.backward(d_act, d_traj, single, pair, seqm, save)

        ms = timed(step, args.steps, args.warmup)
        prof = profiled(step, args.steps, args.no_kprof)
        out = {"metric": "ms per structure-module fold (8 IPA iterations) fwd+bwd", "value": round(ms, 3),
               "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak",
               "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": {"workload": "fold iterations of BASELINE configs[4] (c_s=384, 12 heads, "
                                      "4/8 points, dropout 0.1)", "L": n, "depth": depth},
               "kernels": kernel_table(prof)}
        print(json.dumps(out))
        return
    if args.workload == "triattn":
        mods = ["triangle_attention_starting_node", "triangle_attention_ending_node"]
        prm = bparams.init_block_params(0, rng, modules=mods, gates="zero")
        wdir = bparams.write_manifest(tempfile.mkdtemp(prefix="bc2n_bench_"), prm)
        pair = torch.randn(n, n, 128, device=dev)
        dout = torch.randn(n, n, 128, device=dev)
        layers = [ops.TriangleAttention(wdir, f"param/block0/{mods[i]}/", per_column=bool(i))
                  for i in range(2)]
        outs = [torch.empty_like(pair) for _ in layers]
        dins = [torch.empty_like(pair) for _ in layers]
        saves = [torch.empty(l.save_bytes(n), dtype=torch.uint8, device=dev) for l in layers]

        def step():
            for l, o, s, d in zip(layers, outs, saves, dins):
                l.forward(pair, pmask, None, out=o, save=s)
                l.backward(pair, pmask, None, s, dout, din=d)

        ms = timed(step, args.steps, args.warmup)
        flops = 2 * triattn_flops(n)
        prof = profiled(step, args.steps, args.no_kprof)
        line = {"metric": METRIC if n == 224 else METRIC.replace("at L=224", f"at L={n}"),
                "value": round(flops / (ms * 1e-3) / 1e12, 3),
                "unit": "TFLOP/s", "higher_is_better": True,
                "config": {"workload": "triangle attention fwd+bwd, starting+ending node "
                                       "(BASELINE configs[1])", "L": n, "c_z": 128, "heads": 4,
                           "head_dim": 32, "masked_residues": 0.1, "flops_per_step": flops}}
        cpu = None if args.no_cpu_baseline else cpu_triattn_baseline(n)
    elif args.workload == "design":
        step, save_bytes = design_step_setup(n, rng, dev, m1)
        ms = timed(step, args.steps, args.warmup)
        prof = profiled(step, args.steps, args.no_kprof)
        line = {"metric": "ms per one-call design step (sequence features + embedder + template "
                          "+ 4 extra + 48 Evoformer + 8-iteration structure module + heads + "
                          "confidence, fwd+bwd)",
                "value": round(ms, 2), "unit": "ms", "higher_is_better": False,
                "config": {"workload": f"one-call design step at L={n} ({n - 64} target + 64 "
                                       "designed), logits in, structure and confidence outputs "
                                       "out, d logits back, dropout on",
                           "L": n, "n_seq": 1, "depths": [2, 4, 48, 8]},
                "save_set_gb": round(save_bytes / 1e9, 2)}
        cpu = None
    elif args.workload == "trimul":
        mods = ["triangle_multiplication_outgoing", "triangle_multiplication_incoming"]
        prm = bparams.init_block_params(0, rng, modules=mods, gates="zero")
        wdir = bparams.write_manifest(tempfile.mkdtemp(prefix="bc2n_bench_"), prm)
        pair = torch.randn(n, n, 128, device=dev)
        dout = torch.randn(n, n, 128, device=dev)
        ones = torch.ones(n, n, device=dev)  # configs[2]: all-ones mask
        layers = [ops.TriangleMultiplication(wdir, f"param/block0/{mods[i]}/", outgoing=(i == 0))
                  for i in range(2)]
        outs = [torch.empty_like(pair) for _ in layers]
        dins = [torch.empty_like(pair) for _ in layers]
        saves = [torch.empty(l.save_bytes(n), dtype=torch.uint8, device=dev) for l in layers]

        def step():
            for l, o, s, d in zip(layers, outs, saves, dins):
                l.forward(pair, ones, None, out=o, save=s)
                l.backward(pair, ones, None, s, dout, din=d)

        ms = timed(step, args.steps, args.warmup)
        flops = 2 * trimul_flops(n)
        prof = profiled(step, args.steps, args.no_kprof)
        line = {"metric": "triangle multiplication fwd+bwd, outgoing + incoming (TFLOP/s)",
                "value": round(flops / (ms * 1e-3) / 1e12, 3),
                "unit": "TFLOP/s", "higher_is_better": True,
                "config": {"workload": "triangle multiplication fwd+bwd, outgoing+incoming "
                                       "(BASELINE configs[2])", "L": n, "c_z": 128, "hidden": 128,
                           "mask": "all ones", "flops_per_step": flops}}
        cpu = None
    else:
        # weights: 48 Evoformer blocks, 4 pair-only extra blocks, 2 template
        # blocks (the same draws tests/test_gpu_trunk_full.py checks)
        evo, extra, tpl = bparams.init_trunk_params(rng)
        root = tempfile.mkdtemp(prefix="bc2n_bench_")
        d_evo = bparams.write_manifest(os.path.join(root, "evo"), evo)
        d_extra = bparams.write_manifest(os.path.join(root, "extra"), extra)
        d_tpl = bparams.write_manifest(os.path.join(root, "tpl"), tpl)
        main_stack = ops.EvoformerStack(d_evo, 48)
        extra_stack = ops.EvoformerStack(d_extra, 4, pair_only=True, c_m=64)
        tpl_stack = ops.TemplatePairStack(d_tpl, 2)

        pair0 = torch.randn(n, n, 128, device=dev)
        msa0 = torch.randn(1, n, 256, device=dev)
        emsa0 = torch.randn(1, n, 64, device=dev)
        emask = torch.zeros(1, n, device=dev)       # the design step's extra MSA mask
        tpl0 = torch.randn(n, n, 64, device=dev)
        ct_pair = torch.randn(n, n, 128, device=dev)
        ct_msa = torch.randn(1, n, 256, device=dev)
        ct_tpl = torch.randn(n, n, 64, device=dev)
        keys = [ops.seed_tensor((0, 11 + i), True, dev) for i in range(3)]
        s_main = torch.empty(main_stack.save_bytes(n, 1), dtype=torch.uint8, device=dev)
        s_extra = torch.empty(extra_stack.save_bytes(n, 1), dtype=torch.uint8, device=dev)
        s_tpl = torch.empty(tpl_stack.save_bytes(n), dtype=torch.uint8, device=dev)
        pe, me = torch.empty_like(pair0), torch.empty_like(emsa0)
        pm, mm = torch.empty_like(pair0), torch.empty_like(msa0)
        to = torch.empty_like(tpl0)

        def step():
            tpl_stack.forward(tpl0, pmask, keys[0], out=to, save=s_tpl)
            extra_stack.forward(pair0, emsa0, pmask, emask, keys[1], save=s_extra,
                                pair_out=pe, msa_out=me)
            main_stack.forward(pe, msa0, pmask, mmask, keys[2], save=s_main, pair_out=pm,
                               msa_out=mm)
            dp, _ = main_stack.backward(ct_pair, ct_msa, pmask, mmask, s_main, keys[2])
            extra_stack.backward(dp, torch.zeros_like(emsa0), pmask, emask, s_extra, keys[1])
            tpl_stack.backward(ct_tpl, pmask, s_tpl, keys[0])

        ms = timed(step, args.steps, args.warmup)
        prof = profiled(step, args.steps, args.no_kprof)
        dom = dominant(prof, n)
        dom_prof = profiled(step, args.steps, args.no_kprof or dom is None, only=dom)
        tri = sum(v[0] for k, v in prof.items() if k.startswith("attn_") or k.startswith("triattn."))
        tm = sum(v[0] for k, v in prof.items() if k.startswith("trimul."))
        n_tri = 2 * (48 + 4) * args.steps
        cfg = "BASELINE configs[3]" if n == 224 else "BASELINE configs[4]'s trunk" if n == 512 else "custom length"
        # BASELINE.json's metric names L = 224; a line at another length says its own
        metric = METRIC if n == 224 else METRIC.replace("at L=224", f"at L={n}")
        line = {"metric": metric, "value": round(ms, 2), "unit": "ms", "higher_is_better": False,
                "config": {"workload": f"design-step trunk fwd+bwd at L={n}: 48 Evoformer + 4 "
                                       f"extra-MSA (pair-only) + 2 template blocks ({cfg})",
                           "L": n, "n_seq": 1, "c_m": 256, "c_z": 128, "c_t": 64,
                           "dropout": [0.15, 0.25], "masked_residues": 0.1},
                "triattn_tflops": round(n_tri * triattn_flops(n) / (tri * 1e-3) / 1e12, 2) if tri else None,
                "trimul_tflops": round(n_tri * trimul_flops(n) / (tm * 1e-3) / 1e12, 2) if tm else None,
                "save_set_gb": round((s_main.numel() + s_extra.numel() + s_tpl.numel()) / 1e9, 2)}
        if not args.no_design:
            # the whole one-call design step around this trunk (logits to
            # d(logits)), timed the same way: a secondary key of the line
            del s_main, s_extra, s_tpl
            torch.cuda.empty_cache()
            dstep, _ = design_step_setup(n, np.random.default_rng(1), dev, m1)
            line["design_step_ms"] = round(timed(dstep, args.steps, args.warmup), 2)
            line["design_recycles"] = DESIGN_RECYCLES
        cpu = None if args.no_cpu_baseline else cpu_trunk_baseline(n)

    if dom_prof is None and prof:
        dom = dominant(prof, n)
        if dom is not None:
            dom_prof = profiled(step, args.steps, args.no_kprof, only=dom)
    out = {"metric": line.pop("metric"), "value": line.pop("value"), "unit": line.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms, 3), "higher_is_better": line.pop("higher_is_better"),
           "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
           "config": line.pop("config"), "roofline": roofline_from(prof, n, dom_prof),
           "cpu_baseline": cpu}
    out.update(line)
    if prof and args.workload in ("trunk", "triattn", "trimul"):
        out["kernel_rooflines"] = kernel_rooflines(prof, n)
    out["kernels"] = kernel_table(prof)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
