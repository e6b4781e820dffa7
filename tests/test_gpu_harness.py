"""GPU test of the attn-bench-style harness: this backend's adapter and the
dense SDPA baseline timed through ``time_kernel`` (in process) and
``run_sweep_isolated`` (one spawned process per adapter), rows in attn-bench's
schema with the speedup columns filled."""

from __future__ import annotations

import math

import pytest
import torch

from treeattention_amd import harness as Hn

pytestmark = pytest.mark.gpu


def test_time_kernel_and_isolated_sweep(monkeypatch, tmp_path):
    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", "8")
    monkeypatch.setenv("TREEATTN_LEAF_BLOCK", "64")
    cfg = Hn.BenchConfig(batch=1, seqlen=2048, nheads=2, head_dim=64, dtype=torch.bfloat16, causal=True)
    print("[case] harness time_kernel tree adapter", flush=True)
    r = Hn.time_kernel(Hn.load_entrypoint("treeattention_amd.api:adapter"), cfg, warmup=2, iters=5)
    assert r.status == "ok", r.error_msg
    assert r.fwd_inference.n == 5 and r.fwd_inference.median_ms > 0 and r.step.median_ms > 0
    assert r.bwd_peak_mem_mb > 0 and not math.isnan(r.step_tflops)
    print("[case] harness isolated sweep", flush=True)
    res = Hn.run_sweep_isolated(["treeattention_amd.api:adapter", "sdpa"], [cfg], warmup=1, iters=3,
                                timeout_s=300)
    assert [x.status for x in res] == ["ok", "ok"], [x.error_msg for x in res]
    rows = Hn.annotate_speedups(res, "sdpa")
    assert rows[0]["kernel"] == "treeattn_mi355x" and rows[0]["speedup_step_vs_sdpa"] > 0
    Hn.write_csv(rows, tmp_path / "results.csv")
    assert (tmp_path / "results.csv").read_text().startswith("kernel,dtype,batch,seqlen")
