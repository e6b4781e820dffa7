"""Benchmark: stochastic tree attention fwd+bwd on one MI355X.

Workload (the config the metric is quoted on):
B=2, L=16384, H=16, D=128, bf16, branching 4, leaf block 64, 16 paths per
query, causal (bottom-right aligned), q/k/v/dout ~ N(0,1) from a seed-0
torch.Generator (drawn in that order), Gumbel uniforms from the in-kernel
counter RNG (seed 0).  One step = forward + backward through the public API
(``tree_attention`` + ``out.backward``).

Prints one JSON line with the headline figure (queries/s over the whole
step), fwd/bwd ms, per-kernel-phase times measured with HIP events on the
launch stream, the roofline of the dominant kernel, the CPU oracle timed on
a bounded sample (``cpu_baseline``) and dense SDPA at the same shape.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CONFIGS = {
    # name: B, L, H, D, dtype, b, LB, S, causal, kind
    "C1": (1, 1024, 4, 64, "float32", 2, 16, 4, False, "normal"),
    "C2": (4, 4096, 16, 64, "bfloat16", 2, 64, 8, False, "normal"),
    "C3": (2, 16384, 16, 128, "bfloat16", 4, 64, 16, True, "normal"),
    "C4": (1, 131072, 8, 128, "bfloat16", 2, 128, 16, False, "scaled"),
    "C5-D32": (8, 8192, 32, 32, "float16", 2, 32, 8, True, "skewed"),
    "C5-D96": (8, 8192, 32, 96, "float16", 2, 32, 8, True, "skewed"),
    # the reference's own tree (binary, one token per leaf, Haar keys: the op-level
    # hierarchical_attention and the adapter's default stochastic tree) at C3's shape
    "REF-16k": (2, 16384, 16, 128, "bfloat16", 2, 1, 16, False, "normal"),
    "REF-64k": (2, 65536, 16, 128, "bfloat16", 2, 1, 16, False, "normal"),
}


def skew(q, k, gen, D):
    """Student-t(3) keys and queries with a shared random direction x3 (the C5 stress inputs)."""
    import torch

    B, L, H, _ = k.shape
    chi = sum(torch.randn((B, L, H, 1), device=k.device, generator=gen) ** 2 for _ in range(3)) / 3
    u = torch.randn(D, device=k.device, generator=gen)
    return (q.float() + 3 * u / u.norm()).to(q.dtype), (k.float() / chi.sqrt()).to(k.dtype)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK = {"bfloat16": 2500.0, "float16": 2500.0, "float32": 157.3}  # dense TFLOP/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-sdpa", action="store_true", help="skip the dense SDPA baseline")
    ap.add_argument("--phases-only", action="store_true", help="only run the per-phase loop (for profilers)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 1 GiB device copy (scale reference for HBM counters)")
    ap.add_argument("--dense-cols", type=int, default=0,
                    help="widest tree level run as dense level tiles (0: the library's defaults)")
    ap.add_argument("--causal", choices=("config", "on", "off"), default="config",
                    help="override the config's causality")
    ap.add_argument("--mode", default="stochastic", choices=("stochastic", "deterministic"),
                    help="deterministic: the exact mode of the reference tree (adapter path, Haar keys) at the "
                         "config's B, L, H, D, dtype and causality (default config C2)")
    args = ap.parse_args()
    if args.mode == "deterministic" and "--config" not in sys.argv:
        args.config = "C2"
    return args


def tree_units(B, L, H, D, e, b, LB, S):
    """Algorithmic bytes / FLOPs per launch of each phase (uniforms generated in-kernel).

    With 16-bit inputs, LB > 1, b = 2 or 4 and T*b <= 32 the leaf backward also computes the tree
    gradient along every sample's path (per sample and depth the b child logits, their share of
    dq and of the child summaries' gradient: 6 b D FLOPs), which the leaf_backward phase then counts."""
    NL = L // LB
    T = round(math.log(NL, b))
    NS = b * (NL - 1) // (b - 1)
    BLHD, BLHS = B * L * H * D, B * L * H * S
    sums = NS * B * H * D * e
    path = e == 2 and LB > 1 and b in (2, 4) and T * b <= 32
    return dict(
        T=T,
        NS=NS,
        pool_bytes=BLHD * e + sums,
        sample_bytes=BLHD * e + sums + BLHS * 12,
        sample_flops=BLHS * T * b * 2 * D,
        leaf_fwd_flops=BLHS * 4 * LB * D,
        leaf_bwd_flops=BLHS * 10 * LB * D + (BLHS * 6 * T * b * D if path else 0),
        fwd_bytes=4 * BLHD * e + BLHS * 8 + 2 * sums,
        bwd_bytes=8 * BLHD * e + BLHS * 8 + 2 * sums,
    )


def read_profile(kind: str, key: str, phase: str, config: str):
    """A figure of `phase`'s main kernel from a committed rocprofv3 counter summary
    ``profiles/<kind>_<config>.md`` (a line ``key[phase]: value``), or None."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{config}.md")
    if not os.path.exists(path):
        return None
    m = re.search(re.escape(key) + r"\[" + re.escape(phase) + r"\]:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def read_traffic(phase: str, config: str):
    """HBM bytes per launch of `phase`'s main kernel (``profiles/traffic_<config>.md``: FETCH_SIZE and
    WRITE_SIZE calibrated by a plain copy), or None."""
    return read_profile("traffic", "traffic_bytes_per_launch", phase, config)


# Queries timed per config by the CPU baseline (all heads of batch element 0, the
# last CPU_QUERIES[c] positions, against the full-length tree, keys and values).
CPU_QUERIES = {"C1": 1024, "C2": 1024, "C3": 512, "C4": 128, "C5-D32": 1024, "C5-D96": 512, "REF-16k": 512,
               "REF-64k": 256}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Every host core this process may use (its affinity set), capped by the
    OMP_NUM_THREADS share the host gives it when that is set."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() else n


def cpu_baseline(name: str, cfg) -> dict:
    """The reference's CPU path (``oracle/cpu_path.py``: torch float32, the
    reference's op order -- per-depth gathers, query-block streaming, the
    explicit streaming backward) on every host core: 1 warmup, then the median
    of 3 of the forward and of the whole step, on a bounded sample of the
    workload (all heads of batch 0, the last ``CPU_QUERIES`` positions, full
    tree)."""
    import numpy as np
    import torch

    from oracle import cpu_path as P
    from oracle import tree_oracle as O

    B, L, H, D, dt, b, LB, S, causal, kind = cfg
    threads = cpu_threads()
    torch.set_num_threads(threads)
    nq = min(L, CPU_QUERIES[name])
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(L, H, D, generator=g) for _ in range(3))
    do = torch.randn(nq, H, D, generator=g)
    if kind == "scaled":
        q, k, v = (x / math.sqrt(D) for x in (q, k, v))
    T = O.tree_depth(L // LB, b)
    per_q = H * S * T * b  # uniforms per position of the (B, L, H, S, T, b) tensor; batch 0
    flat = (L - nq) * per_q + np.arange(nq * per_q)
    U = torch.from_numpy(O.uniforms_at(0, flat).reshape(nq, H, S, T, b))
    mode = "natural" if b != 2 else "compat"
    prob = P.Problem(q[L - nq:], k, v, U, torch.arange(L - nq, L), b, LB, causal, mode)
    fwd_s, step_s = [], []
    for it in range(4):  # 1 warmup + 3 timed
        t0 = time.perf_counter()
        C = P.summaries(prob.k, b, LB, mode)
        idx, w, out = prob.forward(C)
        t1 = time.perf_counter()
        prob.backward(C, idx, w, do)
        t2 = time.perf_counter()
        if it:
            fwd_s.append(t1 - t0)
            step_s.append(t2 - t0)
    fwd_m, step_m = sorted(fwd_s)[1], sorted(step_s)[1]
    frac = nq / (B * L)
    return {"value": round(nq / step_m, 3), "unit": "queries/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "fwd_ms": round(fwd_m * 1e3, 1), "bwd_ms": round((step_m - fwd_m) * 1e3, 1),
            "fraction_of_workload": frac,
            "sample": f"oracle/cpu_path.py (torch float32, the reference's op order: per-depth summary gathers, "
                      f"per-(query, sample) leaf-block gathers, explicit streaming backward) on {threads} threads; "
                      f"batch 0, all {H} heads, the last {nq} of {L} queries against the full {L}-token tree "
                      f"({frac:.2%} of the step's queries); 1 warmup + median of 3; step {step_m:.2f} s"}


def det_main(args) -> int:
    """Deterministic mode on the reference tree: fwd+bwd of the adapter path (Haar keys, exact
    weights over every leaf; 16-bit inputs stream, no (L, N) buffer), plus the streaming forward
    kernel timed alone for its roofline (nominal FLOPs of the two products, q K_nodes^T and W V)."""
    import torch

    from treeattention_amd.function import DeterministicAdapterAttention, det_stream_forward, haar_node_keys

    B, L, H, D, dts, _, _, _, causal, kind = CONFIGS[args.config]
    dtype = getattr(torch, dts)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    q, k, v, do = (torch.randn((B, L, H, D), device=dev, dtype=dtype, generator=gen) for _ in range(4))
    if kind == "scaled":
        q, k, v = (x / math.sqrt(D) for x in (q, k, v))
    elif kind == "skewed":
        q, k = skew(q, k, gen, D)
    for x in (q, k, v):
        x.requires_grad_(True)

    def step():
        q.grad = k.grad = v.grad = None
        DeterministicAdapterAttention.apply(q, k, v, causal).backward(do)

    def fwd():
        with torch.no_grad():
            DeterministicAdapterAttention.apply(q, k, v, causal)

    def timed(fn, n):
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n

    for _ in range(args.warmup):
        step()
    step_ms = timed(step, args.steps)
    fwd_ms = timed(fwd, args.steps)
    with torch.no_grad():
        kn = haar_node_keys(k).to(dtype)
        qd, vd = q.detach(), v.detach()
        run = lambda: det_stream_forward(qd, kn, vd, causal)  # noqa: E731
        run()
        kern_ms = timed(run, max(3, args.steps))
    N = L
    flops = 4.0 * B * H * L * N * D * (0.5 if causal else 1.0)
    achieved = flops / (kern_ms / 1e3) / 1e12
    line = {
        "metric": "deterministic tree-attn fwd+bwd ms & queries/s (reference tree, exact weights)",
        "value": round(B * L / (step_ms / 1e3), 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(step_ms - fwd_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts.replace("bfloat16", "bf16").replace("float16", "fp16").replace("float32", "fp32"),
        "data": "synthetic: q,k,v,dout ~ N(0,1) (torch.Generator seed 0)",
        "config": {"workload": f"{args.config} shape, deterministic mode, reference tree (Haar keys)", "batch": B,
                   "seq_len": L, "heads": H, "head_dim": D, "causal": causal},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_PEAK[dts], "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_PEAK[dts], 4), "traffic": None, "kernel": "det_stream_forward",
                     "kernel_ms": round(kern_ms, 4)},
    }
    print(json.dumps(line))
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus > 1 is not supported",
                          "n_gpus": args.gpus}))
        return 2
    if args.mode == "deterministic":
        return det_main(args)
    import torch

    import treeattention_amd as ta
    from treeattention_amd import _lib
    from treeattention_amd.function import TreeOptions, _prep, _strides, make_problem

    cfg = CONFIGS[args.config]
    if args.causal != "config":
        cfg = cfg[:8] + (args.causal == "on",) + cfg[9:]
    B, L, H, D, dts, b, LB, S, causal, kind = cfg
    dtype = getattr(torch, dts)
    dev = torch.device("cuda:0")
    mode = "natural" if b != 2 else "compat"
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    shape = (B, L, H, D)
    q, k, v, do = (torch.randn(shape, device=dev, dtype=dtype, generator=gen) for _ in range(4))
    if kind == "scaled":
        q, k, v = (x / math.sqrt(D) for x in (q, k, v))
    elif kind == "skewed":
        q, k = skew(q, k, gen, D)
    q.requires_grad_(True)
    k.requires_grad_(True)
    v.requires_grad_(True)
    kw = dict(num_samples=S, branching=b, leaf_block=LB, tree_mode=mode, seed=0, dense_cols=args.dense_cols)

    def step():
        q.grad = k.grad = v.grad = None
        out = ta.tree_attention(q, k, v, causal, None, **kw)
        out.backward(do)

    def fwd():
        with torch.no_grad():
            ta.tree_attention(q, k, v, causal, None, **kw)

    def timed(fn, n):
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(n):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / n

    res = {}
    if not args.phases_only:
        for _ in range(args.warmup):
            step()
        t0 = time.perf_counter()
        step_ms = timed(step, args.steps)
        wall = time.perf_counter() - t0
        fwd_ms = timed(fwd, args.steps)
        res.update(step_ms=step_ms, fwd_ms=fwd_ms, wall=wall)

    # ---- per-phase timing through the C ABI (HIP events on the launch stream)
    lib = _lib.load()
    opts = TreeOptions(causal=causal, layout="bshd", **kw)
    qd, kd, vd, dod = (_prep(x.detach()) for x in (q, k, v, do))
    prob = make_problem(qd, kd, vd, opts)
    rec_b, fws_b, bws_b = _lib.byte_sizes(prob)
    out = torch.empty_like(qd)
    w = torch.empty((B, L, H, S), device=dev, dtype=torch.float32)
    prob.w_strides[:] = _strides(w, "bshd")
    rec = torch.empty(rec_b, device=dev, dtype=torch.uint8)
    fws = torch.empty(fws_b, device=dev, dtype=torch.uint8)
    bws = torch.empty(bws_b, device=dev, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    pp = ctypes.byref(prob)
    stream = torch.cuda.current_stream(dev).cuda_stream
    phases = [
        ("pool", lambda: lib.ta_pool(pp, kd.data_ptr(), rec.data_ptr(), stream)),
        ("sample", lambda: lib.ta_sample(pp, qd.data_ptr(), None, 0, w.data_ptr(), rec.data_ptr(), stream)),
        ("bucket", lambda: lib.ta_bucket(pp, rec.data_ptr(), stream)),
        ("leaf_forward", lambda: lib.ta_leaf_forward(pp, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(),
                                                     rec.data_ptr(), fws.data_ptr(), stream)),
        ("leaf_backward", lambda: lib.ta_leaf_backward(pp, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                                       dod.data_ptr(), rec.data_ptr(), dv.data_ptr(),
                                                       bws.data_ptr(), stream)),
        ("tree_backward", lambda: lib.ta_tree_backward(pp, qd.data_ptr(), w.data_ptr(), rec.data_ptr(),
                                                       dq.data_ptr(), dk.data_ptr(), bws.data_ptr(), stream)),
    ]
    n_ph = max(1, args.steps)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(n_ph)]
    for it in range(1 + n_ph):  # first pass is warmup
        for i, (name, fn) in enumerate(phases):
            if it > 0:
                evs[it - 1][i].record()
            _lib.check(fn())
        if it > 0:
            evs[it - 1][-1].record()
    torch.cuda.synchronize()
    phase_ms = {name: sum(evs[j][i].elapsed_time(evs[j][i + 1]) for j in range(n_ph)) / n_ph
                for i, (name, _) in enumerate(phases)}
    if args.copy_calibration:
        src = torch.empty(1 << 29, device=dev, dtype=torch.bfloat16)  # 1 GiB read + 1 GiB written
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_calibration_bytes"] = src.numel() * src.element_size()
    if args.phases_only:
        print(json.dumps({"phase_ms": phase_ms}))
        return 0

    e = torch.finfo(dtype).bits // 8
    u = tree_units(B, L, H, D, e, b, LB, S)
    peak_t = MFMA_PEAK[dts]
    kern = {
        "leaf_backward": ("mfma", u["leaf_bwd_flops"]),
        "leaf_forward": ("mfma", u["leaf_fwd_flops"]),
        "sample": ("hbm", u["sample_bytes"]),
        "pool": ("hbm", u["pool_bytes"]),
    }
    dom = max((k_ for k_ in kern), key=lambda k_: phase_ms[k_])
    bound, units = kern[dom]
    t_s = phase_ms[dom] / 1e3
    if bound == "mfma":
        achieved, peak, unit = units / t_s / 1e12, peak_t, "TFLOP/s"
    else:
        achieved, peak, unit = units / t_s / 1e9, HBM_PEAK_GBS, "GB/s"
    roofline = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": read_traffic(dom, args.config), "kernel": dom}
    if bound == "mfma":
        # the same fraction by counters (profiles/mfma_<config>.md): issued MFMA flops / duration / peak,
        # and the matrix cores' busy share of SIMD-cycles
        roofline["frac_counter"] = read_profile("mfma", "mfma_counter_frac", dom, args.config)
        roofline["mfma_util_pct_counter"] = read_profile("mfma", "mfma_util_pct", dom, args.config)
    per_phase = {}
    for name, (bd, un) in kern.items():
        ts = phase_ms[name] / 1e3
        per_phase[name] = (f"{un / ts / 1e12:.1f} TFLOP/s ({un / ts / 1e12 / peak_t:.1%} of MFMA peak)" if bd == "mfma"
                           else f"{un / ts / 1e9:.0f} GB/s ({un / ts / 1e9 / HBM_PEAK_GBS:.1%} of HBM peak)")

    sdpa = None
    if not args.no_sdpa and dtype != torch.float32:
        try:
            import torch.nn.functional as F
            from torch.nn.attention import SDPBackend, sdpa_kernel

            qs, ks, vs = (x.detach().transpose(1, 2).requires_grad_(True) for x in (q, k, v))
            gs = do.transpose(1, 2)

            def sdpa_step():
                qs.grad = ks.grad = vs.grad = None
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    o = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal)
                o.backward(gs)

            for _ in range(2):
                sdpa_step()
            sdpa = {"ms_per_step": round(timed(sdpa_step, max(3, args.steps // 2)), 3), "backend": "flash/efficient"}
        except Exception as ex:  # no fused backend for this shape
            sdpa = {"skipped": str(ex)[:200]}

    # practical HBM ceiling of this GPU: a plain 1 GiB device copy (1 GiB read + 1 GiB written)
    src = torch.empty(1 << 29, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    copy_ms = min(timed(lambda: dst.copy_(src), 1) for _ in range(5))
    copy_gbs = 2 * src.numel() * src.element_size() / (copy_ms / 1e3) / 1e9
    del src, dst

    cpu = None if args.no_cpu else cpu_baseline(args.config, cfg)
    step_ms = res["step_ms"]
    line = {
        "metric": "tree-attn fwd+bwd ms & queries/s at L=16k bf16; achieved HBM GB/s %peak",
        "value": round(B * L / (step_ms / 1e3), 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "fwd_ms": round(res["fwd_ms"], 4),
        "bwd_ms": round(step_ms - res["fwd_ms"], 4),
        "query_heads_per_s": round(B * L * H / (step_ms / 1e3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts.replace("bfloat16", "bf16").replace("float16", "fp16").replace("float32", "fp32"),
        "data": "synthetic: q,k,v,dout ~ N(0,1) (torch.Generator seed 0), in-kernel Philox uniforms seed 0",
        "config": {"workload": f"{args.config}: stochastic tree attention fwd+bwd", "batch": B, "seq_len": L,
                   "heads": H, "head_dim": D, "branching": b, "leaf_block": LB, "num_samples": S,
                   "causal": causal, "tree_mode": mode},
        "phase_ms": {k_: round(v_, 4) for k_, v_ in phase_ms.items()},
        "phase_roofline": per_phase,
        "roofline": roofline,
        "hbm_copy_GBs": round(copy_gbs, 1),
        "cpu_baseline": cpu,
        "gpu_vs_cpu": round((B * L / (step_ms / 1e3)) / cpu["value"], 1) if cpu else None,
        "sdpa_baseline": sdpa,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
