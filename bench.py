"""Benchmark of the MI355X gated delta rule: the drop-in's forward + backward at BASELINE config 1.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--config 1|2|3|4] [--hv 16|32] [--grouped]
                    [--packed uniform|ragged] [--stored] [--producers] [--ceilings]

A step = one call of macai.gated_delta.chunk_gated_delta_rule (use_qk_l2norm_in_kernel=True, bf16 q/k/v, fp32 g and
beta) followed by its backward for a seeded upstream gradient dO (torch.autograd.grad, so no gradient accumulation),
on synthetic inputs already resident in HBM.  The headline runs the library's default, the reference's: the forward
keeps only its inputs and the backward reruns prep and recomputes the chunk states (op.RECOMPUTE_STATES = True,
BASELINE config 1 as specified).  The stored-states mode (the forward keeps prep's operands and the chunk states) is
timed the same way and reported beside it (--stored swaps the two).  Prints ONE JSON line (rank 0).  Beside the step
time it times every pass inside steps identical to the timed ones with HIP events on the launch stream
(macai.gated_delta.op.EVENTS; the roofline of the dominant kernel) and, for comparison, each pass alone (back-to-back
repeats, whose inputs stay in the Infinity Cache), and the reference's torch path on the host CPU (the oracle's
restatement of transformers' torch_chunk_gated_delta_rule, float32, autograd backward) over the whole config, as a
reported baseline.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mac-ai-engineering_amd"))

import torch  # noqa: E402

METRIC = "gated-delta fwd+bwd tokens/s (B4×T1024,H16,d128 bf16); % HBM/MFMA roofline"
HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
MFMA_PEAK = {"bf16": 2.5e15, "f32": 157.3e12}
PUBLISHED = 401.1e3        # the reference's own published fwd+bwd tokens/s at this config (M3 Max, recompute mode)
C = 64
# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of `bench.py --no-alone --no-cpu`, each
# counter scaled by what it reads for a plain device copy of known size (bench.py --copy-mib 256): FETCH_SIZE x 2.000,
# WRITE_SIZE x 1.000.  Keyed by the config and the mode the profile ran, and stamped with the fingerprint of the
# kernel sources it was taken on: measured_traffic() reports the figures only while the sources still match.
TRAFFIC = {
    (1, "recompute"): {"sources": "1877ef28d2c86210", "bytes": {
        "prep_fwd": 143438156, "state_fwd_out": 110347883, "prep_bwd": 151791475, "state_pair": 313916852,
        "chunk_bwd": 295137910}},
    (1, "stored"): {"sources": "1877ef28d2c86210", "bytes": {
        "prep_fwd": 151858527, "state_fwd_out": 193178324, "state_bwd": 164486517, "chunk_bwd": 295147279}},
}
# the rule's kernel sources and the build script that sets their compile flags (paths under mac-ai-engineering_amd/)
KERNEL_SOURCES = ("csrc/gdr_kernels.hip", "csrc/gdr_common.h", "csrc/gdr_lds.h", "csrc/gdr_stage.h",
                  "csrc/gdr_chunk_bwd8.hip", "build.py")


def kernel_code(text: str) -> str:
    """C++ source without its comments and blank lines, each line stripped: what the compiler sees, so that an edit
    of comments or layout alone keeps the fingerprint (no string literal in these sources holds a comment marker)."""
    import re
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return "\n".join(line.strip() for line in text.splitlines() if line.strip())


def kernel_fingerprint():
    """sha256 (first 16 hex digits) of the rule's kernel sources (their code: kernel_code) and of the build script
    (whole), in KERNEL_SOURCES order."""
    import hashlib
    h = hashlib.sha256()
    for f in KERNEL_SOURCES:
        with open(os.path.join(ROOT, "mac-ai-engineering_amd", f), encoding="utf-8") as fh:
            text = fh.read()
        h.update((text if f.endswith(".py") else kernel_code(text)).encode())
    return h.hexdigest()[:16]


def measured_traffic(cfg, mode):
    """{kernel: HBM bytes per launch} from TRAFFIC for (cfg, mode) while the kernel sources match the profile's,
    with "_source" saying which (or why none)."""
    rec = TRAFFIC.get((cfg, mode))
    if rec is None:
        return {"_source": "no profile of this config and mode"}
    if rec["sources"] != kernel_fingerprint():
        return {"_source": f"stale: the kernels changed since the profile (sources {rec['sources']})"}
    return dict(rec["bytes"], _source=f"rocprofv3 --pmc, kernel sources {rec['sources']}")


CONFIGS = {
    1: dict(B=4, T=1024, Hk=16, Hv=16, DK=128, DV=128, s0=False),
    2: dict(B=2, T=1024, Hk=16, Hv=32, DK=128, DV=128, s0=True),
    3: dict(B=1, T=32768, Hk=16, Hv=16, DK=128, DV=128, s0=False),     # Hv 16 or 32 (--hv)
    4: dict(B=64, T=1, Hk=16, Hv=32, DK=128, DV=128, s0=True),
}


def make_inputs(cfg, seed, dev, on_device=False, **over):
    """The measurement plan's synthetic inputs (q, k, v, u_g, x_g, x_beta, s0, dO drawn in that order in float64);
    keyword overrides replace config fields.  on_device: the same distributions drawn in float32 by the device's own
    generator (seconds faster for config 3's 32,768-token rows; other values, the same workload)."""
    c = dict(CONFIGS[cfg], **over)
    B, T, Hk, Hv, DK, DV = c["B"], c["T"], c["Hk"], c["Hv"], c["DK"], c["DV"]
    rep = Hv // Hk
    where = dev if on_device else "cpu"
    gen = torch.Generator(device=where).manual_seed(seed)
    fdt = torch.float32 if on_device else torch.float64
    randn = lambda *shape: torch.randn(*shape, generator=gen, dtype=fdt, device=where)
    q = randn(B, T, Hk, DK).repeat_interleave(rep, 2)
    k = randn(B, T, Hk, DK).repeat_interleave(rep, 2)
    v = randn(B, T, Hv, DV)
    u = torch.rand(Hv, generator=gen, dtype=fdt, device=where) * math.log(16.0)
    xg = randn(B, T, Hv)
    xb = randn(B, T, Hv)
    g = -torch.exp(u) * torch.nn.functional.softplus(xg)
    beta = torch.sigmoid(xb)
    s0 = randn(B, Hv, DK, DV) * 0.02 if c["s0"] else None
    do = randn(B, T, Hv, DV)
    bf = torch.bfloat16
    out = dict(query=q.to(dev, bf), key=k.to(dev, bf), value=v.to(dev, bf), g=g.to(dev, torch.float32),
               beta=beta.to(dev, torch.float32), initial_state=None if s0 is None else s0.to(dev, torch.float32),
               do=do.to(dev, bf))
    return out, c


def kernel_costs(B, T, H, DK, DV, es=2, Hk=None, chunks=None, keep=False, segs=1):
    """Algorithmic bytes (each declared input read once, each output written once, from argument sizes), split into
    reads and writes, and dense FLOPs (2 per multiply-add, triangular products counted dense) per launch of each
    kernel of the training step.  Hk: key heads of q and k when they come unrepeated (grouped value heads); H by
    default.  chunks: chunks per head over the batch (B ceil(T / 64) by default; packed rows chunk each sequence on
    its own).  keep: the forward's prep also writes A and its state pass S_c and Vn (the stored-states mode: the
    backward then runs neither prep nor the recompute pass).  segs: segments a row's forward runs side by side (the
    map pass reads W, U, Ke, GL and writes each segment's [A | B]; the scan composes them)."""
    Hk = Hk or H
    chunks = chunks or B * math.ceil(T / C)
    n = H * chunks                       # chunk-heads
    tok = B * T * H
    io_k, io_v = tok * DK * es, tok * DV * es
    io_kk = B * T * Hk * DK * es         # one of q, k as the kernels read them
    gb = tok * 4 * 2                     # g and beta
    cdk, cdv, cc = C * DK, C * DV, C * C
    sdk = DK * DV * 4                    # one fp32 state
    pre = 3 * cdk * es + cdv * 4 + cc * es + 4      # prep's row-major outputs W, Ke, Qg, U, M, GL
    inp = 2 * io_kk + io_v + gb                       # q, k, v, g, beta
    prep_flops = n * (2 * 2 * cc * DK + cc * C / 3 + 2 * cc * DK + 2 * cc * DV)
    state_flops = n * (3 * 2 * C * DK * DV + 2 * cc * DV)
    rw = {
        # the forward: prep (A too when keep), then the state pass reads W, U, Ke, GL, Qg, M and writes o (and S_c,
        # Vn when keep)
        "prep_fwd": (inp, n * (pre + (cc * es if keep else 0)), prep_flops),
        "state_fwd_out": (n * pre, io_v + (n * (sdk + cdv * es) if keep else 0), state_flops),
        # the backward: prep with A; the recompute pass reads W, U, Ke, GL and writes S_c (fp32) and Vn; the reverse
        # pass reads Ke, Qg, W, M, GL, dO and writes dS_{c+1} (fp32) and dVn
        "prep_bwd": (inp, n * (pre + cc * es), prep_flops),
        "state_fwd_store": (n * (2 * cdk * es + cdv * 4 + 4), n * (sdk + cdv * es), n * (2 * 2 * C * DK * DV)),
        "state_bwd": (n * (3 * cdk * es + cc * es + 4) + io_v, n * (sdk + cdv * es), state_flops),
        # the per-chunk backward reads q, k, v, g, beta, dO, A, S_c, dS_{c+1}, Vn, dVn; writes dq, dk, dv, dg, dbeta
        "chunk_bwd": (inp + io_v + n * (cc * es + 2 * sdk + 2 * cdv * es), 2 * io_k + io_v + gb,
                      n * (3 * 2 * C * DK * DV + 2 * cc * DK + 3 * 2 * cc * DK + 2 * 2 * cc * DV + 2 * 2 * cc * C
                           + 3 * 2 * cc * DK + 2 * cc * DV)),
        # grouped heads: each of dq, dk folded from per-value-head rows (read H heads, write Hk)
        "group_sum": (io_k, io_kk, tok * DK),
    }
    # the recompute and reverse passes in one launch (macai_gdr_state_pair)
    rw["state_pair"] = tuple(a + b for a, b in zip(rw["state_fwd_store"], rw["state_bwd"]))
    if segs > 1:
        maps = B * (segs - 1) * H * DK * (DK + DV) * 4    # the last segment's map is not needed
        nm = n - B * H * (math.ceil(T / C) - (segs - 1) * math.ceil(math.ceil(T / C) / segs))
        rw["state_map"] = (nm * (2 * cdk * es + cdv * 4 + 4), maps, nm * 2 * 2 * C * DK * (DK + DV))
        rw["state_scan"] = (maps + B * H * sdk, B * segs * H * sdk, B * (segs - 1) * H * 2 * DK * DK * DV)
    return {k: dict(bytes=r + w, reads=r, writes=w, flops=f) for k, (r, w, f) in rw.items()}


def step_kernels(keep, grouped=False):
    """The launches of one training step in order: the stored-states mode (keep) runs prep with A and the state
    pass storing S_c, Vn, then the reverse pass and the chunk backward; the recompute mode runs prep and the output
    pass, then prep with A, the pair pass and the chunk backward."""
    ks = (["prep_fwd", "state_fwd_out", "state_bwd", "chunk_bwd"] if keep
          else ["prep_fwd", "state_fwd_out", "prep_bwd", "state_pair", "chunk_bwd"])
    return ks + (["group_sum", "group_sum"] if grouped else [])


def time_kernels(inp, reps=20, keep=False):
    """Each pass of the step alone: HIP events on the current (launch) stream around `reps` back-to-back launches.
    keep: the forward's prep writes A too and its state pass stores S_c, Vn (the training forward keeps them for the
    backward)."""
    from macai.gated_delta import _native as N
    from macai.gated_delta import op
    q, k, v, g, beta, do = (inp[n] for n in ("query", "key", "value", "g", "beta", "do"))
    s0 = inp["initial_state"]
    B, T, H, DK = q.shape
    DV = v.shape[-1]
    NT = math.ceil(T / C)
    dev, dt = q.device, q.dtype
    f32 = torch.float32
    code, st = N.dtype_code(dt), N.stream_of(q)
    sc = DK ** -0.5
    split = op.split_for(B * H, T, DV)
    split2 = op.split_for(B * H, T, DV, 2)
    e = lambda *shape, d=dt: torch.empty(*shape, device=dev, dtype=d)
    W, U, Ke, GL, Qg, M = e(B, H, NT, C, DK), e(B, H, NT, C, DV, d=f32), e(B, H, NT, C, DK), e(B, H, NT, d=f32), \
        e(B, H, NT, C, DK), e(B, H, NT, C, C)
    A = e(B, H, NT, C, C)
    o = torch.empty_like(v)
    Sc, Vn = e(B, H, NT, DK, DV, d=f32), e(B, H, NT, C, DV)
    dSn, dVn, ds0 = e(B, H, NT, DK, DV, d=f32), torch.empty_like(Vn), e(B, H, DK, DV, d=f32)
    dq, dk, dv, dg, db = (torch.empty_like(x) for x in (q, k, v, g, beta))
    P = N.ptr
    calls = {
        "prep_fwd": ("macai_gdr_prep", P(q), P(k), P(v), P(g), P(beta), P(W), P(U), P(Ke), P(GL), P(Qg), P(M),
                     P(A) if keep else None, B, T, H, H, DK, DV, code, 1, sc, None, 0, st),
        "state_fwd_out": ("macai_gdr_state_fwd", P(W), P(U), P(Ke), P(GL), P(Qg), P(M), P(s0), P(o), None,
                          P(Sc) if keep else None, P(Vn) if keep else None, B, T, H, DK, DV, code,
                          N.STORE_STATES if keep else 0, split, None, 0, st),
        "prep_bwd": ("macai_gdr_prep", P(q), P(k), P(v), P(g), P(beta), P(W), P(U), P(Ke), P(GL), P(Qg), P(M), P(A),
                     B, T, H, H, DK, DV, code, 1, sc, None, 0, st),
        "state_fwd_store": ("macai_gdr_state_fwd", P(W), P(U), P(Ke), P(GL), None, None, P(s0), None, None, P(Sc),
                            P(Vn), B, T, H, DK, DV, code, N.STORE_STATES | N.NO_OUTPUT, split, None, 0, st),
        "state_bwd": ("macai_gdr_state_bwd", P(Ke), P(Qg), P(W), P(M), P(GL), P(do), None, P(dSn), P(dVn), P(ds0),
                      B, T, H, DK, DV, code, split, None, 0, st),
        "state_pair": ("macai_gdr_state_pair", P(W), P(U), P(Ke), P(Qg), P(M), P(GL), P(s0), P(do), None, P(Sc), P(Vn),
                       P(dSn), P(dVn), P(ds0), B, T, H, DK, DV, code, split2, None, 0, st),
        "chunk_bwd": ("macai_gdr_chunk_bwd", P(q), P(k), P(v), P(g), P(beta), P(do), P(A), P(Sc), P(dSn),
                      P(Vn), P(dVn), P(dq), P(dk), P(dv), P(dg), P(db), B, T, H, H, DK, DV, code, 1, sc, None, 0, st),
    }
    order = ["prep_fwd", "state_fwd_out", "prep_bwd", "state_fwd_store", "state_bwd", "state_pair", "chunk_bwd"]
    for name in order:                   # warm, and produce every input of the later passes
        N.call(*calls[name])
    torch.cuda.synchronize()
    out = {}
    for name in order:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            N.call(*calls[name])
        e1.record()
        e1.synchronize()
        out[name] = e0.elapsed_time(e1) / reps * 1e-3     # seconds per launch
    return out, split


def cpu_info():
    """(CPU model, physical cores, CPUs this process may run on, the thread share the environment grants):
    /proc/cpuinfo's model name and distinct (physical id, core id) pairs, the affinity mask, OMP_NUM_THREADS."""
    model, cores, phys = "unknown", set(), None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model == "unknown":
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    cores.add((phys, val))
    except OSError:
        pass
    allowed = len(os.sched_getaffinity(0))
    physical = len(cores) or allowed
    share = int(os.environ.get("OMP_NUM_THREADS") or allowed)
    return model, physical, allowed, share


def cpu_baseline(cfg, threads=0):
    """The reference's torch path (the oracle's restatement of transformers' algorithm at C = 64, float32, the
    solve_triangular inverse, autograd backward) on the host CPU over the whole config, the measurement plan's way
    (bench/bench_gated_delta.py:28, 43-83): 2 warm-up calls, then the median of 5, forward alone and forward +
    backward, with every core the process is granted (physical cores, capped by the CPUs it may run on and by the
    OMP_NUM_THREADS share a GPU box gives one GPU) and with one thread."""
    sys.path.insert(0, ROOT)
    from oracle import gdr
    model, physical, allowed, share = cpu_info()
    n = threads or max(1, min(physical, allowed, share))
    c = dict(CONFIGS[cfg])
    inp = gdr.make_inputs(c["B"], c["T"], c["Hk"], c["Hv"], c["DK"], c["DV"], torch.float32, c["s0"],
                          seed=1000 + cfg)
    leaves = [inp[x].clone().requires_grad_(True) for x in ("query", "key", "value", "g", "beta")]

    def fwd():
        with torch.no_grad():
            gdr.torch_chunk_gated_delta_rule(*leaves, initial_state=inp["initial_state"], output_final_state=True,
                                             use_qk_l2norm_in_kernel=True, inverse="solve")

    def fwd_bwd():
        o, _ = gdr.torch_chunk_gated_delta_rule(*leaves, initial_state=inp["initial_state"], output_final_state=True,
                                                use_qk_l2norm_in_kernel=True, inverse="solve")
        torch.autograd.grad(o, leaves, inp["do"].float())

    def median(fn):
        for _ in range(2):
            fn()
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[2]

    old = torch.get_num_threads()
    try:
        torch.set_num_threads(n)
        t_fb, t_f = median(fwd_bwd), median(fwd)
        torch.set_num_threads(1)
        t1_fb, t1_f = median(fwd_bwd), median(fwd)
    finally:
        torch.set_num_threads(old)
    tok = c["B"] * c["T"]
    return {"value": round(tok / t_fb, 1), "unit": "tokens/s", "cores": n, "kind": "port",
            "sample": f"the whole of config {cfg} (B={c['B']}, T={c['T']}, H={c['Hv']}, D={c['DK']}), fp32 fwd+bwd, "
                      f"median of 5 after 2 warm-ups, {n} threads",
            "ms_fwd_bwd": round(t_fb * 1e3, 2), "ms_fwd": round(t_f * 1e3, 2),
            "fwd_tokens_per_s": round(tok / t_f, 1),
            "one_thread": {"ms_fwd_bwd": round(t1_fb * 1e3, 2), "ms_fwd": round(t1_f * 1e3, 2),
                           "tokens_per_s": round(tok / t1_fb, 1), "fwd_tokens_per_s": round(tok / t1_f, 1)},
            "cpu_model": model, "physical_cores": physical, "cpus_allowed": allowed, "omp_share": share}


def _events_time(fn, reps):
    """Seconds per call of fn: HIP events on the current stream around reps back-to-back calls (after one warm call)."""
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def bench_prefill(args):
    print(json.dumps(prefill_line(args.hv, args.steps, args.warmup)), flush=True)


def prefill_line(hv, steps, warmup, on_device=False):
    """one row of 32,768 tokens, forward only (no_grad: no per-chunk states kept), the final state
    returned; Hv value heads over 16 key heads (q and k unrepeated).  The bound is the 512-chunk chain of the state
    pass; the line reports the value split it ran with and each pass's in-step time."""
    from macai.gated_delta import chunk_gated_delta_rule, op
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    inp, c = make_inputs(3, 1003, dev, on_device=on_device, Hv=hv)
    rep = c["Hv"] // c["Hk"]
    q, k = (inp[n][:, :, ::rep].contiguous() for n in ("query", "key"))
    v, g, beta = inp["value"], inp["g"], inp["beta"]

    def fwd():
        with torch.no_grad():
            return chunk_gated_delta_rule(q, k, v, g, beta, output_final_state=True, use_qk_l2norm_in_kernel=True)
    for _ in range(warmup):
        fwd()
    sec = _events_time(fwd, steps)
    op.EVENTS = []
    for _ in range(min(steps, 10)):
        fwd()
    torch.cuda.synchronize()
    t = {}
    for name, a, b in op.EVENTS:
        t.setdefault(name, []).append(a.elapsed_time(b) * 1e-3)
    op.EVENTS = None
    t = {name: sum(v) / len(v) for name, v in t.items()}
    B, T, H, DK, DV = c["B"], c["T"], c["Hv"], c["DK"], c["DV"]
    segs = op.segments_for(B, T, H, DV)
    cost = kernel_costs(B, T, H, DK, DV, Hk=c["Hk"], segs=segs)
    kernels = {n: {"us": round(x * 1e6, 2), "GB/s": round(cost[n]["bytes"] / x / 1e9, 1),
                   "hbm_frac": round(cost[n]["bytes"] / x / HBM_PEAK, 4)} for n, x in t.items()}
    st = t["state_fwd_out"]
    line = {"metric": f"gated-delta forward tokens/s (B1xT32768, Hv{H}, Hk16, d128 bf16, forward only)",
            "value": round(B * T / sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "BASELINE config 3: long single-row prefill, forward only", "B": B, "T": T,
                       "Hk": c["Hk"], "Hv": H, "DK": DK, "DV": DV, "chunk": C, "segments": segs,
                       "value_split": op.split_for(B * segs * H, T, DV)},
            "roofline": {"kernel": "state_fwd_out", "timing": "in-step HIP events", "bound": "hbm",
                         "achieved": round(cost["state_fwd_out"]["bytes"] / st / 1e9, 1), "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": round(cost["state_fwd_out"]["bytes"] / st / HBM_PEAK, 4),
                         "traffic": None},
            "chain_us_per_chunk": round(st * 1e6 / math.ceil(math.ceil(T / C) / segs), 3),
            "kernels": kernels}
    return line


def decode_bytes(B, H, Hk, DK, DV, es=2):
    """Algorithmic bytes of one decode step: the fp32 state read and written once, q and k at their Hk key heads, v
    and o at the H value heads (es bytes an element), g and beta in fp32."""
    return 2 * B * H * DK * DV * 4 + B * (2 * Hk * DK + 2 * H * DV) * es + B * H * 4 * 2


def bench_decode(args):
    print(json.dumps(decode_line(args.steps, args.warmup)), flush=True)


def decode_line(steps, warmup):
    """one decode step per sequence (B = 64, Hv = 32 over Hk = 16, fp32 state [64, 32, 128, 128]),
    through the drop-in (transformers' torch_recurrent_gated_delta_rule signature) and as the bare C-ABI launch on
    preallocated buffers.  The step reads and writes the whole fp32 state once: HBM-bound, reported against peak."""
    from macai.gated_delta import _native as N
    from macai.gated_delta import recurrent_gated_delta_rule
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    inp, c = make_inputs(4, 1004, dev)
    rep = c["Hv"] // c["Hk"]
    q, k = (inp[n][:, :, ::rep].contiguous() for n in ("query", "key"))
    v, g, beta, s0 = inp["value"], inp["g"], inp["beta"], inp["initial_state"]
    B, H, Hk, DK, DV = c["B"], c["Hv"], c["Hk"], c["DK"], c["DV"]

    def dropin():
        with torch.no_grad():
            return recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0, output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    o = torch.empty(B, 1, H, DV, device=dev, dtype=v.dtype)
    s1 = torch.empty_like(s0)
    P = N.ptr
    st = N.stream_of(q)
    args_k = ("macai_gdr_decode", P(q), P(k), P(v), P(g), P(beta), P(s0), P(o), P(s1), B, H, Hk, DK, DV,
              N.dtype_code(v.dtype), 1, DK ** -0.5, st)
    for _ in range(warmup):
        dropin()
    sec_dropin = _events_time(dropin, steps)
    sec = _events_time(lambda: N.call(*args_k), steps)
    nbytes = decode_bytes(B, H, Hk, DK, DV)
    line = {"metric": "gated-delta decode step GB/s (B64, Hv32, Hk16, d128; fp32 state read + write)",
            "value": round(nbytes / sec / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "BASELINE config 4: one recurrent decode step per sequence", "B": B, "T": 1,
                       "Hk": Hk, "Hv": H, "DK": DK, "DV": DV},
            "roofline": {"kernel": "decode", "timing": "HIP events, C-ABI launches on preallocated buffers",
                         "bound": "hbm", "achieved": round(nbytes / sec / 1e9, 1), "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": round(nbytes / sec / HBM_PEAK, 4), "traffic": None},
            "bytes_per_step": nbytes, "tokens_per_s": round(B / sec, 1),
            "dropin_ms_per_step": round(sec_dropin * 1e3, 4), "dropin_tokens_per_s": round(B / sec_dropin, 1)}
    return line


def bench_producers(cfg, reps=20):
    """The rule's producers at the config's layer widths (key_dim = Hk DK, value_dim = Hv DV): the convolution path
    forward (q, k at key heads, v in x's dtype: the layout the rule reads without copies), its backward (without and
    with the taps' gradient), and the gates forward and backward.  Each entry point is launched `reps` times back to
    back through the C ABI on preallocated buffers and timed with HIP events (the gates' kernels are shorter than a
    launch's host cost, so their event time is a ceiling: rocprof gives their durations), beside the PyTorch path
    (conv1d with groups = channels + silu + split) in the same dtype.  Algorithmic bytes: every input read once and
    every output written once."""
    from macai.gated_delta import _native as N
    c = CONFIGS[cfg]
    dev = torch.device("cuda", 0)
    B, T, Hk, Hv, DK, DV = c["B"], c["T"], c["Hk"], c["Hv"], c["DK"], c["DV"]
    kd, vd, rep = Hk * DK, Hv * DV, Hv // Hk
    C = 2 * kd + vd
    bf, f32 = torch.bfloat16, torch.float32
    gen = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *sh, dt=bf: torch.randn(*sh, device=dev, generator=gen).to(dt)
    x, w4 = rnd(B, T, C), rnd(C, 4, dt=f32) * 0.3
    q, k, v = rnd(B, T, Hk, DK), rnd(B, T, Hk, DK), rnd(B, T, Hv, DV)
    dq, dk, dv, dx = rnd(B, T, Hk, DK), rnd(B, T, Hk, DK), rnd(B, T, Hv, DV), torch.empty(B, T, C, device=dev,
                                                                                          dtype=bf)
    dwp = torch.empty(N.lib().macai_gdr_conv_partials(B, T, C), device=dev, dtype=f32)
    dw = torch.empty(C, 4, device=dev, dtype=f32)
    b, a, A_log, dt = rnd(B, T, Hv), rnd(B, T, Hv), torch.zeros(Hv, device=dev), torch.zeros(Hv, device=dev)
    beta, g, dbeta, dg = (rnd(B, T, Hv, dt=f32) for _ in range(4))
    db, da, dA, ddt = rnd(B, T, Hv), rnd(B, T, Hv), torch.empty(Hv, device=dev), torch.empty(Hv, device=dev)
    P, st, BF = N.ptr, N.stream_of(x), N.BF16
    n = B * T * Hv
    calls = {
        "conv_fwd": (("macai_gdr_conv_fwd", P(x), P(w4), P(q), P(k), P(v), B, T, C, kd, DK, 1, DV, BF, BF, st),
                     2 * B * T * C * 2),
        "conv_bwd": (("macai_gdr_conv_bwd", P(x), P(w4), P(dq), P(dk), P(dv), P(dx), None, None, B, T, C, kd, DK, 1,
                      DV, BF, BF, st), 3 * B * T * C * 2),
        "conv_bwd_dw": (("macai_gdr_conv_bwd", P(x), P(w4), P(dq), P(dk), P(dv), P(dx), P(dwp), P(dw), B, T, C, kd,
                         DK, 1, DV, BF, BF, st), 3 * B * T * C * 2 + 2 * dwp.numel() * 4),
        "gates_fwd": (("macai_gdr_gates_fwd", P(b), P(a), P(A_log), P(dt), P(beta), P(g), n, Hv, BF, st),
                      n * (2 * 2 + 2 * 4)),
        "gates_bwd": (("macai_gdr_gates_bwd", P(b), P(a), P(A_log), P(dt), P(dbeta), P(dg), P(db), P(da), None, None,
                       n, Hv, BF, st), n * (2 * 2 + 2 * 4 + 2 * 2)),
    }

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    wt = w4.to(bf).reshape(C, 1, 4)

    def torch_conv():
        y = torch.nn.functional.silu(torch.nn.functional.conv1d(x.transpose(1, 2), wt, padding=3, groups=C)[..., :T])
        return torch.split(y.transpose(1, 2), [kd, kd, vd], dim=-1)

    res = {}
    for name, (args, nbytes) in calls.items():
        t = timed(lambda: N.call(*args))
        res[name] = {"us": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                     "hbm_frac": round(nbytes / t / HBM_PEAK, 4), "bytes": nbytes}
    res["conv_fwd"]["torch_path_us"] = round(timed(torch_conv) * 1e6, 2)
    line = {"metric": "gated-delta producers: conv+SiLU path and gates, GB/s of algorithmic bytes", "unit": "GB/s",
            "value": res["conv_fwd"]["GB/s"], "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
            "data": "synthetic", "config": {"workload": f"layer producers at BASELINE config {cfg} widths", "B": B,
                                           "T": T, "C": C, "key_dim": kd, "value_dim": vd,
                                           "layout": "q, k at key heads, bf16 v"},
            "roofline": {"kernel": "conv_fwd", "bound": "hbm", "achieved": res["conv_fwd"]["GB/s"],
                         "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": res["conv_fwd"]["hbm_frac"]},
            "kernels": res}
    print(json.dumps(line))


def bench_ceilings(args, mib=1024, reps=10):
    """The device's own streaming rates (macai_gdr_probe_stream: read-only, write-only and copy over `mib` MiB in
    16-byte units, grid-stride; the best of a few workgroup counts, each timed with HIP events over `reps` launches),
    its matrix cores' throughput (macai_gdr_probe_mfma: back-to-back MFMAs of the kernels' bf16 and fp32 shapes and
    the larger bf16 one, the best of a few workgroup counts), and the floor the streams put under the config's
    training step: every kernel's algorithmic reads at the read rate plus its writes at the write rate, summed over the
    step's launches (the recompute mode and the stored-states mode)."""
    from macai.gated_delta import _native as N
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    nbytes = mib << 20
    src = torch.ones(nbytes // 4, device=dev)
    dst = torch.empty_like(src)
    st = N.stream_of(src)
    rates = {}
    for mode, name, moved in ((0, "read", nbytes), (1, "write", nbytes), (2, "copy", 2 * nbytes)):
        best = None
        for blocks in (1024, 2048, 4096, 8192, 16384):
            sec = _events_time(lambda: N.call("macai_gdr_probe_stream", mode, N.ptr(src), N.ptr(dst), nbytes, blocks,
                                              st), reps)
            if best is None or sec < best[0]:
                best = (sec, blocks)
        rates[name] = {"GB/s": round(moved / best[0] / 1e9, 1), "blocks": best[1], "us": round(best[0] * 1e6, 2)}
    mfma = {}
    out = torch.empty(16384 * 256, device=dev)
    for mode, name, peak in ((0, "bf16 16x16x32", MFMA_PEAK["bf16"]), (1, "f32 16x16x4", MFMA_PEAK["f32"]),
                             (2, "bf16 32x32x16", MFMA_PEAK["bf16"])):
        best = None
        for blocks in (1024, 2048, 4096):
            iters = 4096 if mode != 1 else 2048
            sec = _events_time(lambda: N.call("macai_gdr_probe_mfma", mode, iters, N.ptr(out), blocks, st), 3)
            fl = N.lib().macai_gdr_probe_mfma_flops(mode, iters, blocks) / sec
            if best is None or fl > best[0]:
                best = (fl, blocks, sec)
        mfma[name] = {"TFLOP/s": round(best[0] / 1e12, 1), "of_peak": round(best[0] / peak, 4),
                      "peak_TFLOP/s": peak / 1e12, "blocks": best[1], "us": round(best[2] * 1e6, 1)}
    c = CONFIGS[args.config]
    floors = {}
    for mode, keep in (("recompute", False), ("stored", True)):
        cost = kernel_costs(c["B"], c["T"], c["Hv"], c["DK"], c["DV"], keep=keep)
        ks = step_kernels(keep)
        reads = sum(cost[k]["reads"] for k in ks)
        writes = sum(cost[k]["writes"] for k in ks)
        floors[mode] = {"reads_MB": round(reads / 1e6, 1), "writes_MB": round(writes / 1e6, 1),
                        "floor_us": round((reads / (rates["read"]["GB/s"] * 1e9)
                                           + writes / (rates["write"]["GB/s"] * 1e9)) * 1e6, 1),
                        "floor_us_at_peak": round((reads + writes) / HBM_PEAK * 1e6, 1)}
    line = {"metric": "device streaming ceilings (GB/s) and the training step's algorithmic-byte floor",
            "value": rates["copy"]["GB/s"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "data": "synthetic", "config": {"workload": f"{mib} MiB streams; step floor of BASELINE config "
                                                        f"{args.config}"},
            "peak": HBM_PEAK / 1e9, "rates": rates, "mfma": mfma, "step_floor": floors}
    print(json.dumps(line), flush=True)


def make_step(cfg, dev, grouped=False, packed=None):
    """A training step of config cfg: the drop-in's forward (use_qk_l2norm_in_kernel=True) and torch.autograd.grad
    for the seeded dO over every leaf (q and k at the model's key heads, v, g, beta and the initial state when the
    config has one).  grouped: with Hk < Hv, q and k go to the rule unrepeated; otherwise the step repeats them first,
    as the model does.  packed: "uniform" / "ragged" runs the B rows as one packed row (cu_seqlens).  Returns (step,
    config, the drop-in's extra keywords, the inputs)."""
    from macai.gated_delta import chunk_gated_delta_rule
    inp, c = make_inputs(cfg, 1000 + cfg, dev)
    rep = c["Hv"] // c["Hk"]
    # q, k leaves at the model's key heads (make_inputs draws them per key head and repeats)
    kq = {n: inp[n][:, :, ::rep].contiguous() for n in ("query", "key")}
    leaves = [kq["query"], kq["key"]] + [inp[n] for n in ("value", "g", "beta")]
    kw = {}
    if packed:                                # the B rows as one row of B * T tokens
        Bp, Tp = c["B"], c["T"]
        leaves = [x.reshape(1, Bp * Tp, *x.shape[2:]) for x in leaves]
        inp["do"] = inp["do"].reshape(1, Bp * Tp, *inp["do"].shape[2:])
        if packed == "uniform":
            lens = [Tp] * Bp
        else:                                 # 4 B seeded lengths summing to B * T
            gen = torch.Generator().manual_seed(7)
            w = torch.rand(4 * Bp, generator=gen) + 0.01
            lens = (w / w.sum() * Bp * Tp).long().clamp_min(1).tolist()
            lens[-1] += Bp * Tp - sum(lens)
        kw["cu_seqlens"] = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
        if inp["initial_state"] is not None:
            inp["initial_state"] = None       # one state per sequence would be needed; the packed runs start at zero
    leaves = [x.requires_grad_(True) for x in leaves]
    s0 = inp["initial_state"]
    if s0 is not None:
        s0.requires_grad_(True)
        leaves.append(s0)
    do = inp["do"]

    def step():
        q, k = leaves[0], leaves[1]
        if rep > 1 and not grouped:               # the model's layout: repeat over each group first
            q, k = q.repeat_interleave(rep, 2), k.repeat_interleave(rep, 2)
        o, _ = chunk_gated_delta_rule(q, k, *leaves[2:5], initial_state=s0, output_final_state=False,
                                      use_qk_l2norm_in_kernel=True, **kw)
        return torch.autograd.grad(o, leaves, do)
    return step, c, kw, inp


def other_configs(step1, steps=20, warmup=3):
    """The default line's compact figures beside the headline: config 1's step on the float32 kernels
    (op.BF16_OPERANDS = False, the reference's own precision) and with the forward keeping prep's operands for the
    backward, which then recomputes only the chunk states (op.KEEP_PREP), config 2's training step (q, k repeated by the step as
    the model does, and grouped), config 3's forward at Hv 16 and 32 (inputs drawn on the device) and config 4's
    decode step, each timed the way its own --config line times it, with fewer steps."""
    from macai.gated_delta import op
    dev = torch.device("cuda", 0)
    ns = argparse.Namespace(steps=steps, warmup=warmup)
    out = {}
    old = op.BF16_OPERANDS
    try:
        op.BF16_OPERANDS = False
        sec, in_step = _time_step(step1, ns)
    finally:
        op.BF16_OPERANDS = old
    B1, T1 = CONFIGS[1]["B"], CONFIGS[1]["T"]
    out["config1_f32_compute"] = {"ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(B1 * T1 / sec, 1),
                                  "kernels_us": {n: round(t * 1e6, 2) for n, t in in_step.items()}}
    old = op.KEEP_PREP, op.RECOMPUTE_STATES
    try:
        op.KEEP_PREP, op.RECOMPUTE_STATES = True, True
        sec, in_step = _time_step(step1, ns)
    finally:
        op.KEEP_PREP, op.RECOMPUTE_STATES = old
    out["config1_kept_prep"] = {"ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(B1 * T1 / sec, 1),
                                "kernels_us": {n: round(t * 1e6, 2) for n, t in in_step.items()}}
    for grouped in (False, True):
        step, c, _, _ = make_step(2, dev, grouped)
        sec, _ = _time_step(step, ns)
        out["config2_" + ("grouped" if grouped else "repeated")] = {
            "ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(c["B"] * c["T"] / sec, 1)}
        del step
    for hv in (16, 32):
        ln = prefill_line(hv, steps, warmup, on_device=True)
        out[f"config3_hv{hv}"] = {"ms_fwd": ln["ms_per_step"], "tokens_per_s": ln["value"],
                                  "segments": ln["config"]["segments"], "value_split": ln["config"]["value_split"],
                                  "state_pass_us": ln["kernels"]["state_fwd_out"]["us"],
                                  "state_pass_hbm_frac": ln["roofline"]["frac"]}
        torch.cuda.empty_cache()
    ln = decode_line(steps, warmup)
    out["config4_decode"] = {"us": round(ln["ms_per_step"] * 1e3, 2), "GB/s": ln["value"],
                             "hbm_frac": ln["roofline"]["frac"], "tokens_per_s": ln["tokens_per_s"],
                             "dropin_us": round(ln["dropin_ms_per_step"] * 1e3, 2)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS),
                    help="1 (the headline), 2: fwd+bwd steps; 3: the long prefill, forward only; 4: one decode step")
    ap.add_argument("--hv", type=int, default=16, choices=[16, 32], help="config 3's value heads")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--stored", action="store_true",
                    help="headline the stored-states mode (the forward keeps prep's operands and the chunk states, "
                         "op.RECOMPUTE_STATES = False) instead of the reference's default, where the backward reruns "
                         "prep and recomputes the chunk states; the other mode is always reported beside it")
    ap.add_argument("--recompute", action="store_true", help="the default (kept for old command lines)")
    ap.add_argument("--ceilings", action="store_true",
                    help="measure the device's streaming read / write / copy rates and the config's step floor at "
                         "those rates instead of the rule")
    ap.add_argument("--grouped", action="store_true",
                    help="configs with Hk < Hv: q and k go to the rule unrepeated (grouped value heads); without "
                         "it the "
                         "step repeats them first, as the model does (repeat_interleave inside the timed step)")
    ap.add_argument("--packed", choices=["uniform", "ragged"],
                    help="run the batch as one packed row (cu_seqlens): B sequences of T tokens, or seeded ragged "
                         "lengths with the same total")
    ap.add_argument("--producers", action="store_true",
                    help="time the rule's producers (the convolution path and the gates) instead of the rule")
    ap.add_argument("--f32-compute", action="store_true",
                    help="run the bf16 inputs on the float32 kernels (op.BF16_OPERANDS = False, the reference's own "
                         "precision) and report that step's time only")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave out the default line's compact figures of configs 2-4 and of config 1 on the float32 "
                         "kernels")
    ap.add_argument("--no-alone", action="store_true",
                    help="skip timing each pass alone, so a kernel trace of the run holds the step's launches only")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (calibrates rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the gated delta rule has no cross-GPU step in this build "
              "(head/batch sharding needs no collective); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.ceilings:
        bench_ceilings(args)
        return
    if args.producers:
        bench_producers(args.config)
        return
    if args.config == 3:
        bench_prefill(args)
        return
    if args.config == 4:
        bench_decode(args)
        return
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    step, c, kw, inp = make_step(args.config, dev, args.grouped, args.packed)

    from macai.gated_delta import op
    if args.f32_compute:
        old = op.BF16_OPERANDS
        try:
            op.BF16_OPERANDS = False
            sec, in_step = _time_step(step, args)
        finally:
            op.BF16_OPERANDS = old
        line = {"metric": METRIC + ", bf16 inputs on the float32 kernels", "value": round(c["B"] * c["T"] / sec, 1),
                "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": "f32", "data": "synthetic",
                "config": {"workload": f"gated-delta drop-in fwd+bwd, BASELINE config {args.config}, "
                                       "op.BF16_OPERANDS = False", "B": c["B"], "T": c["T"], "Hv": c["Hv"],
                           "DK": c["DK"], "DV": c["DV"], "recompute_prep_in_backward": op.RECOMPUTE_STATES},
                "kernels": {n: {"us": round(t * 1e6, 2)} for n, t in in_step.items()}}
        print(json.dumps(line), flush=True)
        return
    default_mode = op.RECOMPUTE_STATES
    modes = [not args.stored, args.stored]           # headline first, then the other mode as a second field
    runs = []
    try:
        for recompute in modes:
            op.RECOMPUTE_STATES = recompute
            runs.append(_time_step(step, args))
    finally:
        op.RECOMPUTE_STATES = default_mode
    (sec, in_step), (sec_other, in_step_other) = runs
    keep = args.stored
    B, T, H, DK, DV = c["B"], c["T"], c["Hv"], c["DK"], c["DV"]
    tokens = B * T

    # each pass alone at the batched layout; packed rows (whose per-sequence chunking those launches do not follow)
    # report the in-step times only
    rows = B * H if not args.packed else (len(kw["cu_seqlens"]) - 1) * H
    if args.packed or args.no_alone:
        alone, split = {}, op.split_for(rows, T, DV)
    else:
        alone, split = time_kernels(inp, keep=keep)
    if args.copy_mib:
        src = torch.ones(args.copy_mib << 18, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
    chunks = None
    if args.packed:
        cu = kw["cu_seqlens"].tolist()
        chunks = sum(math.ceil((b - a) / C) for a, b in zip(cu, cu[1:]))
    cost = kernel_costs(B, T, H, DK, DV, Hk=c["Hk"] if args.grouped else None, chunks=chunks, keep=keep)
    traffic = measured_traffic(args.config, "stored" if keep else "recompute") if not args.packed else {}
    kernels = {}
    for name, t in in_step.items():
        bw = cost[name]["bytes"] / t
        fl = cost[name]["flops"] / t
        kernels[name] = {"us": round(t * 1e6, 2), "us_alone": round(alone[name] * 1e6, 2) if name in alone else None,
                         "GB/s": round(bw / 1e9, 1), "hbm_frac": round(bw / HBM_PEAK, 4),
                         "TFLOP/s": round(fl / 1e12, 2), "mfma_frac": round(fl / MFMA_PEAK["bf16"], 4),
                         "traffic": traffic.get(name)}
    dom = max(in_step, key=in_step.get)
    bw = cost[dom]["bytes"] / in_step[dom]
    roof = {"kernel": dom, "timing": "in-step HIP events", "bound": "hbm", "achieved": round(bw / 1e9, 1),
            "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(bw / HBM_PEAK, 4), "traffic": traffic.get(dom),
            "algorithmic_bytes": cost[dom]["bytes"], "traffic_source": traffic.get("_source")}
    value = tokens / sec
    other_cost = kernel_costs(B, T, H, DK, DV, Hk=c["Hk"] if args.grouped else None, chunks=chunks, keep=not keep)
    other = {"recompute_prep_in_backward": keep, "ms_per_step": round(sec_other * 1e3, 4),
             "tokens_per_s": round(tokens / sec_other, 1),
             "kernels": {n: {"us": round(t * 1e6, 2), "hbm_frac": round(other_cost[n]["bytes"] / t / HBM_PEAK, 4)}
                         for n, t in in_step_other.items()}}
    line = {"metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": round(value / PUBLISHED, 2) if args.config == 1 and not keep and not args.packed else None,
            "dtype": "bf16", "data": "synthetic",
            "config": {"workload": f"gated-delta drop-in fwd+bwd, BASELINE config {args.config}", "B": B, "T": T,
                       "Hk": c["Hk"], "Hv": H, "DK": DK, "DV": DV, "chunk": C, "l2norm_in_kernel": True,
                       "qk_heads_to_the_rule": c["Hk"] if args.grouped else H,
                       "packed_rows": None if not args.packed else {"mode": args.packed,
                                                                     "sequences": len(kw["cu_seqlens"]) - 1,
                                                                     "chunks_per_head": chunks},
                       "initial_state": c["s0"], "value_split": split,
                       "pair_split": None if keep else op.split_for(rows, T, DV, 2),
                       "overlapped_state_passes": (not keep) and op.pairs_states(torch.bfloat16), "recompute_prep_in_backward": not keep},
            "roofline": roof, "kernels": kernels,
            "stored_states" if not keep else "recompute_states": other}
    if args.config == 1 and not (args.no_configs or args.packed or args.grouped or args.stored):
        line["configs"] = other_configs(step, min(args.steps, 20), min(args.warmup, 3))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.config, args.cpu_threads)
    print(json.dumps(line), flush=True)


def _time_step(step, args):
    """(seconds per step, {pass: seconds in the step}) for the current op settings: W warm-up steps, K steps timed
    with HIP events and the wall clock (the larger counts), then up to 20 further identical steps with HIP events on
    the launch stream around every launch (op.EVENTS; an event record costs the stream ~4 us, so the timed steps
    carry none)."""
    from macai.gated_delta import op
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu = e0.elapsed_time(e1) * 1e-3
    op.EVENTS = []
    try:
        for _ in range(min(args.steps, 20)):
            step()
        torch.cuda.synchronize()
        in_step = {}
        for name, a, b in op.EVENTS:
            in_step.setdefault(name, []).append(a.elapsed_time(b) * 1e-3)
    finally:
        op.EVENTS = None
    return max(wall, gpu) / args.steps, {name: sum(ts) / len(ts) for name, ts in in_step.items()}


if __name__ == "__main__":
    main()
