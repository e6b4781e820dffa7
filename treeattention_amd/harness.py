"""Benchmark harness with attn-bench's protocol and result schema.

A counterpart of ``packages/attn-bench/src/attn_bench/harness.py``,
``reporting.py`` and the output part of ``run.py``, so tree-attention numbers
from this backend land in the same CSV / JSON / meta files as the reference's
sweeps:

* ``time_kernel`` follows ``harness.py:299-480``: compatibility check, inputs
  ``randn`` from a device generator seeded with ``seed`` in the order q, k, v,
  grad (``harness.py:163-171``); pass 1 times the inference forward under
  ``no_grad``, pass 2 the training step (forward + ``out.backward(grad)``),
  each after warmup iterations that watch the allocator for per-iteration
  growth; inputs must keep their storage (``adapters.py:135-154``); then three
  untimed memory probes (forward peak, memory kept for backward, step peak).
  Timing is CUDA events around each iteration, back to back, no cleanup in the
  timed loop (``harness.py:207-221``).
* ``TimingStats`` / ``Result.row`` / ``write_csv`` / ``write_json`` /
  ``annotate_speedups`` keep the reference's field names, statistics
  (population std, ``p10 = sorted[int(0.1 (n-1))]``) and speedup columns.
* ``run_sweep_isolated`` runs each adapter in its own spawned process
  (``harness.py:669-750``): results stream back through a queue ending in a
  sentinel; a child that dies is reported as ``error`` for its remaining
  configs; after an OOM the larger sequence lengths of that adapter are
  skipped.
* FLOPs follow the FlashAttention convention of ``flops.py`` (``4 b h s^2 d``,
  halved when causal, backward 2.5x) so TFLOP/s columns compare across
  kernels; for tree attention they are nominal (dense-equivalent) numbers.

Adapters are ``pkg.module:attr`` entry points (``adapters.py:61-93``) that
return a ``KernelAdapter``; ``"sdpa"`` names the built-in PyTorch
``scaled_dot_product_attention`` baseline.
"""

from __future__ import annotations

import argparse
import csv
import datetime as dt
import importlib
import json
import math
import os
import statistics
import subprocess
import sys
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Callable, Iterable, Optional

import torch

PRIMARY_BASELINE = "sdpa"

_DTYPES = {"fp16": torch.float16, "float16": torch.float16, "half": torch.float16, "bf16": torch.bfloat16,
           "bfloat16": torch.bfloat16, "fp32": torch.float32, "float32": torch.float32}


def parse_dtype(name) -> torch.dtype:
    if isinstance(name, torch.dtype):
        return name
    key = str(name).lower().strip()
    if key not in _DTYPES:
        raise ValueError(f"unknown dtype {name!r}; expected one of {sorted(_DTYPES)}")
    return _DTYPES[key]


def dtype_str(dtype: torch.dtype) -> str:
    return {torch.float16: "fp16", torch.bfloat16: "bf16", torch.float32: "fp32"}.get(dtype, str(dtype))


@dataclass(frozen=True)
class BenchConfig:
    """One benchmark point (``configs.py:44-64``)."""

    batch: int
    seqlen: int
    nheads: int
    head_dim: int
    dtype: torch.dtype
    causal: bool

    def to_dict(self) -> dict:
        d = asdict(self)
        d["dtype"] = dtype_str(self.dtype)
        return d

    @property
    def label(self) -> str:
        return (f"b={self.batch} s={self.seqlen} h={self.nheads} d={self.head_dim} "
                f"dtype={dtype_str(self.dtype)} causal={self.causal}")


def build_sweep(*, batches=(1,), nheads_list=(2,), head_dims=(64,), seqlens=tuple(1 << e for e in range(11, 21)),
                causals=(False,), dtypes=(torch.bfloat16,)) -> list[BenchConfig]:
    """Cartesian product in the reference's nesting order (dtype, batch, heads, dim, seqlen, causal)."""
    return [BenchConfig(b, s, h, d, dt_, c) for dt_ in dtypes for b in batches for h in nheads_list
            for d in head_dims for s in seqlens for c in causals]


# ---------------------------------------------------------------- FLOPs ----

def fwd_flops(batch: int, seqlen: int, nheads: int, head_dim: int, causal: bool) -> float:
    """Nominal attention forward FLOPs: two ``s x s x d`` products per (batch, head), causal halves."""
    f = 4.0 * batch * nheads * seqlen * seqlen * head_dim
    return f * 0.5 if causal else f


def bwd_flops(batch: int, seqlen: int, nheads: int, head_dim: int, causal: bool) -> float:
    return 2.5 * fwd_flops(batch, seqlen, nheads, head_dim, causal)


def tflops_per_sec(flops: float, elapsed_ms: float) -> float:
    return float("nan") if elapsed_ms <= 0.0 else flops / (elapsed_ms * 1e-3) / 1e12


# -------------------------------------------------------------- results ----

@dataclass
class TimingStats:
    median_ms: float
    mean_ms: float
    std_ms: float
    p10_ms: float
    p90_ms: float
    min_ms: float
    max_ms: float
    n: int

    @classmethod
    def from_samples(cls, samples: list[float]) -> "TimingStats":
        s = sorted(samples)
        n = len(s)
        return cls(median_ms=statistics.median(s), mean_ms=statistics.fmean(s),
                   std_ms=statistics.pstdev(s) if n > 1 else 0.0, p10_ms=s[max(0, int(0.10 * (n - 1)))],
                   p90_ms=s[min(n - 1, int(0.90 * (n - 1)))], min_ms=s[0], max_ms=s[-1], n=n)


@dataclass
class Result:
    kernel: str
    config: BenchConfig
    status: str  # "ok" | "oom" | "skipped" | "error"
    fwd_inference: Optional[TimingStats] = None
    step: Optional[TimingStats] = None
    fwd_inference_tflops: float = float("nan")
    step_tflops: float = float("nan")
    fwd_peak_mem_mb: float = float("nan")
    fwd_saved_mem_mb: float = float("nan")
    bwd_peak_mem_mb: float = float("nan")
    error_msg: str = ""
    skip_reason: str = ""
    extra: dict = field(default_factory=dict)

    def row(self) -> dict:
        """Flat row with the reference's column names (``harness.py:116-160``)."""
        c = self.config
        row = {"kernel": self.kernel, "dtype": dtype_str(c.dtype), "batch": c.batch, "seqlen": c.seqlen,
               "nheads": c.nheads, "head_dim": c.head_dim, "causal": c.causal, "status": self.status}
        for prefix, st, tf in (("fwd_inference", self.fwd_inference, self.fwd_inference_tflops),
                               ("step", self.step, self.step_tflops)):
            if st is not None:
                row.update({f"{prefix}_ms_median": st.median_ms, f"{prefix}_ms_mean": st.mean_ms,
                            f"{prefix}_ms_std": st.std_ms, f"{prefix}_ms_p10": st.p10_ms,
                            f"{prefix}_ms_p90": st.p90_ms, f"{prefix}_tflops": tf})
        if self.status == "ok":
            row.update({"fwd_peak_mem_mb": self.fwd_peak_mem_mb, "fwd_saved_mem_mb": self.fwd_saved_mem_mb,
                        "bwd_peak_mem_mb": self.bwd_peak_mem_mb})
        if self.error_msg:
            row["error_msg"] = self.error_msg
        if self.skip_reason:
            row["skip_reason"] = self.skip_reason
        for k, v in self.extra.items():
            if isinstance(v, (bool, int, float, str)):
                row[k] = v
        return row


# -------------------------------------------------------------- adapters ----

def load_entrypoint(spec: str):
    """``"pkg.module:attr"`` -> the adapter (``attr`` called if it is a factory)."""
    if spec == "sdpa":
        return sdpa_adapter()
    mod, _, attr = spec.partition(":")
    if not mod or not attr:
        raise ValueError(f"entry point must look like 'pkg.module:attr', got {spec!r}")
    obj = getattr(importlib.import_module(mod), attr)
    if callable(obj) and not hasattr(obj, "fn"):
        obj = obj()
    if not hasattr(obj, "fn") or not hasattr(obj, "name"):
        raise TypeError(f"{spec!r} did not give a KernelAdapter")
    return obj


def _sdpa_fn(q, k, v, causal, softmax_scale):
    import torch.nn.functional as F

    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=causal,
                                       scale=softmax_scale)
    return o.transpose(1, 2)


def sdpa_adapter():
    """Dense PyTorch SDPA on bshd tensors (the reported dense baseline)."""
    from .api import KernelAdapter

    return KernelAdapter(name="sdpa", fn=_sdpa_fn, supports_backward=True, supports_causal=True,
                         allowed_dtypes=frozenset({torch.float16, torch.bfloat16}),
                         allowed_head_dims=frozenset({32, 64, 96, 128}), layout="bshd")


def validate_inputs(adapter, q, k, v, dtype) -> None:
    """The kernel contract checks of ``adapters.py:96-132``."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"{name} is not a torch.Tensor")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on the GPU, got {t.device}")
        if t.dtype != dtype:
            raise ValueError(f"{name}.dtype={t.dtype}, expected {dtype}")
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D (b,s,h,d), got shape {tuple(t.shape)}")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"q/k/v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if q.shape[-1] not in adapter.allowed_head_dims:
        raise ValueError(f"head_dim {q.shape[-1]} not supported by {adapter.name}")


# ---------------------------------------------------------------- timing ----

def _make_inputs(cfg: BenchConfig, *, requires_grad: bool, seed: int):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    shape = (cfg.batch, cfg.seqlen, cfg.nheads, cfg.head_dim)
    mk = lambda rg: torch.randn(shape, device="cuda", dtype=cfg.dtype, generator=gen, requires_grad=rg)  # noqa: E731
    return mk(requires_grad), mk(requires_grad), mk(requires_grad), mk(False)


def _warmup(fn, n: int, on_leak, threshold_mb: float) -> None:
    """``n`` warmup calls; after the first, allocator growth beyond ``threshold_mb`` is reported."""
    base = None
    for i in range(n):
        fn()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        now = torch.cuda.memory_allocated()
        if base is None:
            base = now
            continue
        delta = (now - base) / (1024 * 1024)
        if delta > threshold_mb:
            on_leak(i, delta)
            base = now


def _time_iters(fn, iters: int) -> list[float]:
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in ev]


def _peak_mb(fn) -> float:
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    fn()
    torch.cuda.synchronize()
    return (torch.cuda.max_memory_allocated() - base) / (1024 * 1024)


def _saved_mb(fn) -> float:
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    out = fn()
    torch.cuda.synchronize()
    kept = (torch.cuda.memory_allocated() - base) / (1024 * 1024)
    del out
    return kept


def time_kernel(adapter, cfg: BenchConfig, *, warmup: int = 10, iters: int = 50, do_backward: bool = True,
                seed: int = 0, leak_threshold_mb: float = 1.0) -> Result:
    """Time one adapter on one config with the reference's two passes and memory probes."""
    ok, reason = adapter.is_compatible(cfg.dtype, cfg.head_dim, cfg.causal)
    if not ok:
        return Result(kernel=adapter.name, config=cfg, status="skipped", skip_reason=reason)
    if not torch.cuda.is_available():
        return Result(kernel=adapter.name, config=cfg, status="error", error_msg="GPU not available")

    def on_leak(kind):
        def cb(i, delta):
            print(f"[warn] per-iter leak: {adapter.name} s={cfg.seqlen} phase={kind} iter={i} +{delta:.2f} MiB",
                  file=sys.stderr)
        return cb

    want_bwd = do_backward and adapter.supports_backward
    q = k = v = g = None
    try:
        q, k, v, g = _make_inputs(cfg, requires_grad=want_bwd, seed=seed)
        validate_inputs(adapter, q, k, v, cfg.dtype)
        scale = 1.0 / math.sqrt(cfg.head_dim)
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr())
        ff = fwd_flops(cfg.batch, cfg.seqlen, cfg.nheads, cfg.head_dim, cfg.causal)
        bf = bwd_flops(cfg.batch, cfg.seqlen, cfg.nheads, cfg.head_dim, cfg.causal)

        def fwd_inference():
            with torch.no_grad():
                adapter.fn(q, k, v, cfg.causal, scale)

        _warmup(fwd_inference, warmup, on_leak("fwd_inference"), leak_threshold_mb)
        inf = TimingStats.from_samples(_time_iters(fwd_inference, iters))
        if (q.data_ptr(), k.data_ptr(), v.data_ptr()) != ptrs:
            raise ValueError("kernel appears to have replaced storage of q/k/v (data_ptr changed); "
                             "kernels must not modify inputs")

        def reset_grads():
            q.grad = k.grad = v.grad = None

        step = None
        step_tf = float("nan")
        if want_bwd:
            def train_step():
                reset_grads()
                adapter.fn(q, k, v, cfg.causal, scale).backward(g)

            _warmup(train_step, warmup, on_leak("step"), leak_threshold_mb)
            step = TimingStats.from_samples(_time_iters(train_step, iters))
            step_tf = tflops_per_sec(ff + bf, step.median_ms)

        fwd_peak = _peak_mb(lambda: adapter.fn(q, k, v, cfg.causal, scale)) if want_bwd else _peak_mb(fwd_inference)
        torch.cuda.empty_cache()
        reset_grads()
        saved = _saved_mb(lambda: adapter.fn(q, k, v, cfg.causal, scale)) if want_bwd else float("nan")
        torch.cuda.empty_cache()
        reset_grads()
        if want_bwd:
            def step_mem():
                reset_grads()
                adapter.fn(q, k, v, cfg.causal, scale).backward(g)
            bwd_peak = _peak_mb(step_mem)
        else:
            bwd_peak = float("nan")
        torch.cuda.empty_cache()
        reset_grads()
        return Result(kernel=adapter.name, config=cfg, status="ok", fwd_inference=inf, step=step,
                      fwd_inference_tflops=tflops_per_sec(ff, inf.median_ms), step_tflops=step_tf,
                      fwd_peak_mem_mb=fwd_peak, fwd_saved_mem_mb=saved, bwd_peak_mem_mb=bwd_peak)
    except torch.cuda.OutOfMemoryError as e:
        return Result(kernel=adapter.name, config=cfg, status="oom", error_msg=str(e))
    except Exception as e:  # a failing cell is recorded, the sweep goes on
        return Result(kernel=adapter.name, config=cfg, status="error", error_msg=f"{type(e).__name__}: {e}")
    finally:
        del q, k, v, g
        if torch.cuda.is_available():
            torch.cuda.empty_cache()


def _sweep_one(adapter, sweep, kwargs, emit) -> None:
    """One adapter over the sweep; after an OOM the larger sequence lengths are skipped."""
    oom_at = None
    thr = kwargs.get("leak_threshold_mb", 1.0)
    for cfg in sweep:
        if oom_at is not None and cfg.seqlen > oom_at:
            emit(Result(kernel=adapter.name, config=cfg, status="skipped", skip_reason=f"prior OOM at s={oom_at}"))
            continue
        if torch.cuda.is_available():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        before = torch.cuda.memory_allocated() if torch.cuda.is_available() else 0
        t0 = time.perf_counter()
        res = time_kernel(adapter, cfg, **kwargs)
        res.extra["wallclock_s"] = time.perf_counter() - t0
        if torch.cuda.is_available():
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            res.extra["leaked_mb"] = (torch.cuda.memory_allocated() - before) / (1024 * 1024)
            if res.extra["leaked_mb"] > thr:
                print(f"[warn] leak: {adapter.name} s={cfg.seqlen} retained {res.extra['leaked_mb']:.1f} MiB",
                      file=sys.stderr)
        if res.status == "oom":
            oom_at = cfg.seqlen
        emit(res)


def run_sweep(adapters, sweep, *, on_result: Callable | None = None, **kwargs) -> list[Result]:
    """All adapters in this process, in series."""
    out: list[Result] = []

    def emit(r):
        out.append(r)
        if on_result is not None:
            on_result(r)

    for a in adapters:
        _sweep_one(a, sweep, kwargs, emit)
    return out


def _child(spec: str, sweep, kwargs, queue) -> None:
    """Spawned worker: one adapter over the sweep, results streamed, then a None sentinel."""
    try:
        adapter = load_entrypoint(spec)
    except Exception as e:
        for cfg in sweep:
            queue.put(Result(kernel=spec, config=cfg, status="error",
                             error_msg=f"adapter init failed: {type(e).__name__}: {e}"))
        queue.put(None)
        return
    _sweep_one(adapter, sweep, kwargs, queue.put)
    queue.put(None)


def run_sweep_isolated(specs: list[str], sweep, *, on_result: Callable | None = None, timeout_s: float = 3600,
                       **kwargs) -> list[Result]:
    """Each adapter entry point in its own spawned process, in series; its GPU context (and every
    pool it holds) is released when it exits.  A child that dies reports its remaining configs as
    errors."""
    import multiprocessing as mp

    ctx = mp.get_context("spawn")
    out: list[Result] = []
    for spec in specs:
        queue = ctx.Queue()
        proc = ctx.Process(target=_child, args=(spec, sweep, kwargs, queue))
        proc.start()
        got: list[Result] = []
        done = False
        while True:
            try:
                msg = queue.get(timeout=timeout_s)
            except Exception:
                break
            if msg is None:
                done = True
                break
            got.append(msg)
            out.append(msg)
            if on_result is not None:
                on_result(msg)
        proc.join(timeout=30)
        if proc.is_alive():
            proc.terminate()
            proc.join(timeout=5)
        if not done:
            seen = {r.config for r in got}
            for cfg in sweep:
                if cfg in seen:
                    continue
                r = Result(kernel=spec, config=cfg, status="error",
                           error_msg=f"child process exited prematurely (exitcode={proc.exitcode})")
                out.append(r)
                if on_result is not None:
                    on_result(r)
            print(f"[warn] adapter {spec!r} subprocess exited with code {proc.exitcode} before completing sweep",
                  file=sys.stderr)
    return out


# ------------------------------------------------------------- reporting ----

def _speedup(base_ms, cand_ms) -> float:
    if base_ms is None or cand_ms is None or cand_ms <= 0 or math.isnan(base_ms) or math.isnan(cand_ms):
        return float("nan")
    return base_ms / cand_ms


def _key(r: Result) -> tuple:
    c = r.config
    return (c.batch, c.seqlen, c.nheads, c.head_dim, c.dtype, c.causal)


def annotate_speedups(results: list[Result], baseline_name: str = PRIMARY_BASELINE) -> list[dict]:
    """Rows plus ``speedup_{fwd_inference,step}_vs_<baseline>`` where the baseline ran the same config."""
    base = {_key(r): r for r in results if r.kernel == baseline_name and r.status == "ok"}
    rows = []
    for r in results:
        row = r.row()
        b = base.get(_key(r))
        if b is not None and r.kernel != baseline_name and r.status == "ok":
            row["speedup_fwd_inference_vs_" + baseline_name] = _speedup(
                b.fwd_inference.median_ms if b.fwd_inference else None,
                r.fwd_inference.median_ms if r.fwd_inference else None)
            row["speedup_step_vs_" + baseline_name] = _speedup(b.step.median_ms if b.step else None,
                                                               r.step.median_ms if r.step else None)
        rows.append(row)
    return rows


def write_csv(rows: Iterable[dict], path) -> None:
    rows = list(rows)
    if not rows:
        Path(path).write_text("")
        return
    names: list[str] = []
    for r in rows:
        for k in r:
            if k not in names:
                names.append(k)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=names)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def write_json(rows: Iterable[dict], path) -> None:
    Path(path).write_text(json.dumps(list(rows), indent=2, default=str))


def _fmt(x, spec=".3f") -> str:
    if x is None or (isinstance(x, float) and math.isnan(x)):
        return "-"
    return format(x, spec) if isinstance(x, float) else str(x)


def format_table(rows: list[dict], baseline_name: str = PRIMARY_BASELINE) -> str:
    cols = [("kernel", "kernel", None), ("dtype", "dtype", None), ("b", "batch", None), ("s", "seqlen", None),
            ("h", "nheads", None), ("d", "head_dim", None), ("causal", "causal", None), ("status", "status", None),
            ("inf_ms", "fwd_inference_ms_median", ".3f"), ("step_ms", "step_ms_median", ".3f"),
            ("inf_TF/s", "fwd_inference_tflops", ".1f"), ("step_TF/s", "step_tflops", ".1f"),
            ("fwd_mem_MiB", "fwd_peak_mem_mb", ".1f"), ("saved_MiB", "fwd_saved_mem_mb", ".1f"),
            ("bwd_mem_MiB", "bwd_peak_mem_mb", ".1f"),
            (f"sp_inf/{baseline_name}", f"speedup_fwd_inference_vs_{baseline_name}", ".2f"),
            (f"sp_step/{baseline_name}", f"speedup_step_vs_{baseline_name}", ".2f")]
    lines = ["\t".join(c[0] for c in cols)]
    for r in rows:
        lines.append("\t".join(_fmt(r.get(key), spec) if spec else str(r.get(key, "-")) for _, key, spec in cols))
    return "\n".join(lines)


def _git_sha() -> str:
    try:
        return subprocess.run(["git", "rev-parse", "--short", "HEAD"], capture_output=True, text=True,
                              cwd=os.path.dirname(os.path.abspath(__file__)), timeout=10).stdout.strip() or "nogit"
    except Exception:
        return "nogit"


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="attn-bench-style sweep of tree-attention adapters")
    ap.add_argument("--kernel", action="append", default=[],
                    help="adapter entry point 'pkg.module:attr' (repeatable); 'sdpa' for the dense baseline")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--nheads", type=int, default=2)
    ap.add_argument("--head-dims", default="64")
    ap.add_argument("--seqlens", default="2048,4096,8192")
    ap.add_argument("--causal", default="false", help="comma list of true/false")
    ap.add_argument("--dtypes", default="bf16")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--isolate", action="store_true", help="one spawned process per adapter")
    ap.add_argument("--treeattn-num-samples", type=int, default=None)
    ap.add_argument("--output-dir", default="results")
    args = ap.parse_args(argv)
    if args.treeattn_num_samples is not None:
        os.environ["TREEATTN_NUM_SAMPLES"] = str(args.treeattn_num_samples)
    if not torch.cuda.is_available():
        print("ERROR: no GPU available; this harness times GPU kernels.", file=sys.stderr)
        return 2
    specs = args.kernel or ["treeattention_amd.api:adapter", "sdpa"]
    ints = lambda s: [int(x) for x in s.split(",") if x]  # noqa: E731
    sweep = build_sweep(batches=(args.batch,), nheads_list=(args.nheads,), head_dims=ints(args.head_dims),
                        seqlens=ints(args.seqlens), causals=[x.strip().lower() == "true" for x in args.causal.split(",")],
                        dtypes=[parse_dtype(x) for x in args.dtypes.split(",")])
    run_id = f"{dt.datetime.now().strftime('%Y%m%d-%H%M%S')}-{_git_sha()}"
    out_dir = Path(args.output_dir) / run_id
    out_dir.mkdir(parents=True, exist_ok=True)
    adapters_meta = []
    for spec in specs:
        a = load_entrypoint(spec)
        adapters_meta.append({"name": a.name, "entrypoint": spec,
                              "allowed_dtypes": sorted(dtype_str(d) for d in a.allowed_dtypes),
                              "allowed_head_dims": sorted(a.allowed_head_dims),
                              "supports_backward": a.supports_backward, "supports_causal": a.supports_causal})
    meta = {"run_id": run_id, "device": torch.cuda.get_device_name(0), "torch": torch.__version__,
            "hip": torch.version.hip, "warmup": args.warmup, "iters": args.iters, "seed": args.seed,
            "do_backward": not args.no_backward, "isolate": args.isolate,
            "env": {n: os.environ.get(n) for n in ("TREEATTN_NUM_SAMPLES", "TREEATTN_BRANCHING", "TREEATTN_LEAF_BLOCK",
                                                   "TREEATTN_TREE_MODE", "TREEATTN_SEED", "PYTORCH_ROCM_ARCH")},
            "adapters": adapters_meta, "sweep": [c.to_dict() for c in sweep]}
    (out_dir / "meta.json").write_text(json.dumps(meta, indent=2))

    def on_result(r: Result) -> None:
        tag = {"ok": "ok", "oom": "OOM", "skipped": "skip", "error": "ERR"}.get(r.status, r.status)
        line = f"  [{tag:>4}] {r.kernel:<18} s={r.config.seqlen:<7}"
        if r.status == "ok":
            stp = r.step.median_ms if r.step else float("nan")
            line += f" inf={r.fwd_inference.median_ms:8.3f}ms step={stp:8.3f}ms"
        print(line, flush=True)

    kw = dict(warmup=args.warmup, iters=args.iters, do_backward=not args.no_backward, seed=args.seed)
    if args.isolate:
        results = run_sweep_isolated(specs, sweep, on_result=on_result, **kw)
    else:
        results = run_sweep([load_entrypoint(s) for s in specs], sweep, on_result=on_result, **kw)
    rows = annotate_speedups(results, PRIMARY_BASELINE)
    write_csv(rows, out_dir / "results.csv")
    write_json(rows, out_dir / "results.json")
    print(format_table(rows, PRIMARY_BASELINE))
    print(f"[run] wrote {out_dir / 'results.csv'} and results.json, meta.json")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
