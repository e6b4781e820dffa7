"""CPU tests of the attn-bench-style harness (``treeattention_amd/harness.py``).

Statistics, FLOP counts and row/CSV/JSON schemas against the definitions of
attn-bench (``harness.py:74-160``, ``flops.py``, ``reporting.py``) with values
worked out by hand; without a GPU ``time_kernel`` reports an error cell and the
isolated runner streams one result per config from a spawned child.
"""

from __future__ import annotations

import csv
import json
import math

import pytest
import torch

from treeattention_amd import harness as Hn


def test_timing_stats_definitions():
    st = Hn.TimingStats.from_samples([5.0, 1.0, 3.0, 2.0, 4.0])
    assert (st.median_ms, st.mean_ms, st.min_ms, st.max_ms, st.n) == (3.0, 3.0, 1.0, 5.0, 5)
    assert st.std_ms == pytest.approx(math.sqrt(2.0))  # population std
    assert st.p10_ms == 1.0 and st.p90_ms == 4.0       # sorted[int(0.1*4)], sorted[int(0.9*4)]
    one = Hn.TimingStats.from_samples([7.0])
    assert one.std_ms == 0.0 and one.p10_ms == one.p90_ms == 7.0


def test_flop_convention():
    f = Hn.fwd_flops(2, 1024, 4, 64, False)
    assert f == 4.0 * 2 * 4 * 1024 * 1024 * 64
    assert Hn.fwd_flops(2, 1024, 4, 64, True) == f / 2
    assert Hn.bwd_flops(2, 1024, 4, 64, False) == 2.5 * f
    assert Hn.tflops_per_sec(2e12, 1000.0) == 2.0 and math.isnan(Hn.tflops_per_sec(1.0, 0.0))


def _cfg(s=1024):
    return Hn.BenchConfig(batch=1, seqlen=s, nheads=2, head_dim=64, dtype=torch.bfloat16, causal=False)


def test_rows_speedups_and_files(tmp_path):
    st = Hn.TimingStats.from_samples([2.0, 2.0])
    base = Hn.Result(kernel="sdpa", config=_cfg(), status="ok", fwd_inference=st, step=st, fwd_peak_mem_mb=1.0,
                     fwd_saved_mem_mb=0.5, bwd_peak_mem_mb=2.0)
    fast = Hn.Result(kernel="tree", config=_cfg(), status="ok",
                     fwd_inference=Hn.TimingStats.from_samples([0.5]), step=Hn.TimingStats.from_samples([1.0]),
                     extra={"wallclock_s": 1.5, "ignored": [1, 2]})
    skip = Hn.Result(kernel="tree", config=_cfg(2048), status="skipped", skip_reason="dtype")
    rows = Hn.annotate_speedups([base, fast, skip], "sdpa")
    assert list(rows[0])[:8] == ["kernel", "dtype", "batch", "seqlen", "nheads", "head_dim", "causal", "status"]
    assert rows[0]["dtype"] == "bf16" and rows[0]["step_ms_median"] == 2.0 and rows[0]["fwd_peak_mem_mb"] == 1.0
    assert rows[1]["speedup_fwd_inference_vs_sdpa"] == 4.0 and rows[1]["speedup_step_vs_sdpa"] == 2.0
    assert rows[1]["wallclock_s"] == 1.5 and "ignored" not in rows[1]
    assert rows[2]["skip_reason"] == "dtype" and "fwd_peak_mem_mb" not in rows[2]
    Hn.write_csv(rows, tmp_path / "r.csv")
    Hn.write_json(rows, tmp_path / "r.json")
    back = list(csv.DictReader(open(tmp_path / "r.csv")))
    assert len(back) == 3 and back[1]["speedup_step_vs_sdpa"] == "2.0"
    assert json.loads((tmp_path / "r.json").read_text())[2]["status"] == "skipped"
    assert "sp_step/sdpa" in Hn.format_table(rows)


def test_time_kernel_without_gpu_is_an_error_cell():
    a = Hn.sdpa_adapter()
    r = Hn.time_kernel(a, _cfg(), warmup=1, iters=1)
    assert r.status == "error" and "GPU" in r.error_msg
    r = Hn.time_kernel(a, Hn.BenchConfig(1, 64, 1, 48, torch.bfloat16, False))
    assert r.status == "skipped" and "head_dim" in r.skip_reason


def test_entry_points():
    a = Hn.load_entrypoint("treeattention_amd.api:adapter")
    assert a.name == "treeattn_mi355x" and a.supports_backward
    with pytest.raises(ValueError):
        Hn.load_entrypoint("no_colon")


def test_isolated_runner_streams_results_from_a_child():
    sweep = [_cfg(1024), _cfg(2048)]
    seen = []
    res = Hn.run_sweep_isolated(["sdpa", "no.such.module:adapter"], sweep, on_result=seen.append, warmup=1,
                                iters=1, timeout_s=300)
    assert len(res) == 4 and len(seen) == 4
    assert [r.status for r in res[:2]] == ["error", "error"] and "GPU" in res[0].error_msg
    assert all("adapter init failed" in r.error_msg for r in res[2:])


def test_main_refuses_without_gpu(tmp_path):
    assert Hn.main(["--output-dir", str(tmp_path)]) == 2
