"""CPU tests of the host side: the C-ABI library loads, exports what the header
declares, sizes and validates problems (no GPU compute), and the Python
interfaces parse their configuration like the reference adapters."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

import treeattention_amd as ta
from treeattention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions() -> list[str]:
    src = open(os.path.join(ROOT, "include", "treeattn_amd.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"\b(ta_[a-z_]+)\s*\(", src)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 11
    assert set(names) == set(_lib.EXPORTS)
    for n in names:
        assert hasattr(lib, n), n
    assert lib.ta_version() == 1


def _problem(**kw):
    p = _lib.Problem()
    d = dict(B=2, L=16384, H=16, D=128, N=16384, num_samples=16, branching=4, leaf_block=64,
             tree_mode=_lib.TA_TREE_NATURAL, causal=1, dtype=_lib.TA_BF16, scale=0.088, max_logit=1e3)
    d.update(kw)
    for k_, v_ in d.items():
        setattr(p, k_, v_)
    st = (d["L"] * d["H"] * d["D"], d["H"] * d["D"], d["D"])
    for a in ("q_strides", "k_strides", "v_strides", "o_strides", "g_strides", "w_strides"):
        getattr(p, a)[:] = st
    return p


def test_struct_layout_and_sizes():
    assert ctypes.sizeof(_lib.Problem) == 232
    rec, fws, bws = _lib.byte_sizes(_problem())
    BLHS = 2 * 16384 * 16 * 16
    assert fws >= BLHS * 128 * 2  # one bf16 partial row per (query, sample)
    assert rec >= 4 * BLHS * 4  # leaves, slots, weights, order
    ns = _lib.record_offset(_problem(), _lib.TA_REC_NUM_ROWS)
    assert ns == 32 + 32 + 64 + 256  # levels 4, 16, 64, 256 padded to 32 rows


def test_path_rows_layout():
    """16-bit problems with b = 2 or 4 and T*b <= 32 take the tree gradient along each pair's
    path in the leaf backward: the record keeps a copy of the output (dout . out in the backward)
    and the backward workspace drops the dense G^T tiles; dense_cols > 0 keeps the dense
    levels, float inputs and one-token leaves always do."""
    out_e = 2 * 16384 * 16 * 128 * 2             # a bf16 copy of the output
    sum_t = 32 * (32 + 32 + 64 + 256) * 128 * 2  # the dense backward's transposed summaries
    rec_p, fws_p, bws_p = _lib.byte_sizes(_problem())
    rec_d, fws_d, bws_d = _lib.byte_sizes(_problem(dense_cols=1024))
    assert rec_p == rec_d + out_e - sum_t and fws_p == fws_d
    assert bws_p < bws_d
    # C4's shape (128-key blocks, head dim 128, T*b = 20): 32 path rows
    c4 = dict(B=1, L=131072, N=131072, H=8, leaf_block=128, branching=2, causal=0)
    assert _lib.byte_sizes(_problem(**c4))[2] < _lib.byte_sizes(_problem(dense_cols=1024, **c4))[2]
    # T*b > 32 (b = 2 and 17 levels) keeps the dense levels and bands: no float output in the record
    deep = dict(B=1, L=131072 * 2, N=131072 * 2, H=1, leaf_block=2, branching=2, causal=0)
    assert _lib.byte_sizes(_problem(**deep))[0] == _lib.byte_sizes(_problem(dense_cols=1024, **deep))[0]
    f32 = dict(dtype=_lib.TA_F32, D=64)
    assert _lib.byte_sizes(_problem(**f32)) == _lib.byte_sizes(_problem(dense_cols=1024, **f32))


@pytest.mark.parametrize("D,LB", [(128, 64), (96, 64), (96, 128), (64, 128), (32, 128), (128, 128)])
def test_float_leaf_tiles_fit(D, LB):
    """fp32 inputs with large head dims or blocks run the leaf backward with 32- or 16-pair
    tiles (D=128 at LB=128: V read from global memory) instead of being refused."""
    N = LB * 2 ** 8
    _lib.byte_sizes(_problem(dtype=_lib.TA_F32, D=D, leaf_block=LB, N=N, L=N, branching=2, causal=0))


def test_backward_inputs_without_gaps():
    """dq / dk / dv are written with the strides of q / k / v into ``empty_like`` buffers, so
    the backward takes views with gaps (a slice of heads, q inside a fused qkv tensor) as
    contiguous copies and dense layouts (any dim order) as they are."""
    from treeattention_amd.function import _dense

    x = torch.randn(2, 64, 16, 32)
    assert _dense(x) is x
    p = x.permute(1, 0, 2, 3)
    assert _dense(p) is p and torch.empty_like(p).stride() == p.stride()
    for view in (x[:, :, 4:8], torch.randn(2, 64, 3, 16, 32)[:, :, 0], x[:, ::2]):
        d = _dense(view)
        assert d.is_contiguous() and torch.equal(d, view)
        assert torch.empty_like(d).stride() == d.stride()


def test_many_samples_run_in_chunks():
    """More than 64 samples: the record holds one chunk record per <= 64 samples plus every
    sample's leaf block and the float output; workspaces are reused chunk after chunk."""
    one = _lib.byte_sizes(_problem(num_samples=64))
    two = _lib.byte_sizes(_problem(num_samples=128))
    out_e = 2 * 16384 * 16 * 128 * 2    # the single-chunk record's copy of the output
    assert two[0] > 2 * one[0] - out_e  # two chunk records + leaves + float output
    assert two[1] == one[1]             # chunks of 64: the same forward workspace
    assert two[2] > one[2]              # + float accumulators
    lo = _lib.record_offset(_problem(num_samples=128), _lib.TA_REC_LEAVES)
    assert lo + 2 * 16384 * 16 * 128 * 4 <= two[0]
    _lib.byte_sizes(_problem(num_samples=1024))
    _lib.byte_sizes(_problem(num_samples=100, causal=0))
    # the per-phase entry points take one launch's worth
    lib = _lib.load()
    rc = lib.ta_bucket(ctypes.byref(_problem(num_samples=65)), None, None)
    assert rc != 0 and b"ta_forward" in lib.ta_last_error()


@pytest.mark.parametrize("kw,exc", [
    (dict(D=80), NotImplementedError),
    (dict(num_samples=1025), NotImplementedError),
    (dict(num_samples=65, causal=2, branching=2, leaf_block=1, tree_mode=_lib.TA_TREE_COMPAT), NotImplementedError),
    (dict(leaf_block=256), NotImplementedError),
    (dict(N=16384 + 64, L=16384 + 64), ValueError),  # not leaf_block * b^T
    (dict(branching=3), ValueError),
    (dict(tree_mode=_lib.TA_TREE_COMPAT), ValueError),  # compat is binary
    (dict(causal=1, L=20000), ValueError),  # causal needs L <= N
    (dict(dtype=7), ValueError),
    (dict(causal=2), ValueError),  # the reference causal mode needs the reference tree
    (dict(causal=3), ValueError),
])
def test_validation_errors(kw, exc):
    with pytest.raises(exc):
        _lib.byte_sizes(_problem(**kw))
    assert _lib.load().ta_last_error()


def test_resolve_num_samples(monkeypatch):
    monkeypatch.delenv("TREEATTN_NUM_SAMPLES", raising=False)
    assert ta.resolve_num_samples() is None
    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", "0")
    assert ta.resolve_num_samples() is None
    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", " 16 ")
    assert ta.resolve_num_samples() == 16
    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", "x")
    with pytest.raises(ValueError):
        ta.resolve_num_samples()
    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", "-2")
    with pytest.raises(ValueError):
        ta.resolve_num_samples()


def test_tree_config_defaults_are_the_reference_tree(monkeypatch):
    for n in ("TREEATTN_BRANCHING", "TREEATTN_LEAF_BLOCK", "TREEATTN_TREE_MODE", "TREEATTN_SEED"):
        monkeypatch.delenv(n, raising=False)
    assert ta.resolve_tree_config() == dict(branching=2, leaf_block=1, tree_mode="compat", seed=0)
    monkeypatch.setenv("TREEATTN_TREE_MODE", "bogus")
    with pytest.raises(ValueError):
        ta.resolve_tree_config()


def test_adapter_metadata():
    ad = ta.adapter()
    assert ad.layout == "bshd" and ad.supports_backward and ad.supports_causal
    assert ad.is_compatible(torch.bfloat16, 128, True) == (True, "")
    assert not ad.is_compatible(torch.bfloat16, 80, False)[0]


def test_attn_fn_deterministic_mode_checks(monkeypatch):
    # TREEATTN_NUM_SAMPLES unset -> the reference adapter's deterministic mode
    # (baselines/treeattn_torch.py:55-56): power-of-two seqlen, reference tree,
    # device tensors
    monkeypatch.delenv("TREEATTN_NUM_SAMPLES", raising=False)
    x = torch.zeros(1, 16, 1, 32)
    with pytest.raises(ValueError, match="device"):
        ta.attn_fn(x, x, x, False, None)
    y = torch.zeros(1, 12, 1, 32)
    with pytest.raises(ValueError, match="power-of-two"):
        ta.attn_fn(y, y, y, False, None)
    monkeypatch.setenv("TREEATTN_BRANCHING", "4")
    with pytest.raises(ValueError, match="reference tree"):
        ta.attn_fn(x, x, x, False, None)


def test_op_level_mode_and_shape_errors():
    x = torch.zeros(8, 1, 64)
    with pytest.raises(ValueError, match="device"):
        ta.hierarchical_attention(x, x[:7], x, num_heads=2, mode="deterministic")
    with pytest.raises(ValueError, match="mode"):
        ta.hierarchical_attention(x, x[:7], x, num_heads=2, mode="exact")
    with pytest.raises(ValueError):
        ta.hierarchical_attention(x, x[:5], x, num_heads=2)
    with pytest.raises(ValueError):
        ta.hierarchical_attention(x, x[:7], x, num_heads=3)
    with pytest.raises(ValueError, match="num_samples"):
        ta.hierarchical_attention(x, x[:7], x, num_heads=2, num_samples=None)


def test_deterministic_entry_points_validate_before_launching():
    lib = _lib.load()
    # non-power-of-two and oversized leaf counts are refused with a message, nothing is launched
    assert lib.ta_det_weights(None, 11, None, 12, 0, 1, 12, 0, None) == 2
    assert b"2^T" in lib.ta_last_error()
    assert lib.ta_det_grad(None, 65535, None, None, 65536, 1, 65536, 0, None) == 2
    assert lib.ta_det_weights(None, 15, None, 16, 0, 1, 16, 0, None) == 0  # no rows: nothing to do
    assert lib.ta_det_weights(None, 3, None, 16, 16, 16, 16, 0, None) == 1  # row stride too small
    ks = (ctypes.c_int64 * 3)(0, 0, 0)
    assert lib.ta_haar_keys(_lib.TA_BF16, None, ks, None, None, 1, 1, 32, 12, None) == 1
    nb = ctypes.c_int64(0)
    assert lib.ta_haar_workspace_bytes(2, 3, 64, 4096, ctypes.byref(nb)) == 0 and nb.value == 4 * 2 * 3 * 32 * 64


def test_cpu_tensors_are_rejected_not_computed():
    x = torch.zeros(1, 64, 1, 32)
    with pytest.raises(ValueError):
        ta.tree_attention(x, x, x, num_samples=4)


def _ref_tree_problem(L, causal=False):
    from treeattention_amd import _lib

    p = _lib.Problem()
    p.B, p.L, p.H, p.D, p.N = 2, L, 16, 128, L
    p.num_samples, p.branching, p.leaf_block = 16, 2, 1
    p.tree_mode = _lib.TA_TREE_NODEKEYS
    p.causal = _lib.TA_CAUSAL_REFERENCE if causal else _lib.TA_CAUSAL_NONE
    p.dtype, p.scale, p.max_logit = _lib.TA_BF16, 0.1, 1e3
    for f in ("q_strides", "k_strides", "v_strides", "o_strides", "g_strides"):
        getattr(p, f)[:] = (16 * 128, 2 * 16 * 128, 128)  # (L, B, H, D) op-level layout
    p.w_strides[:] = (16 * 16, 2 * 16 * 16, 16)
    return p


@pytest.mark.parametrize("causal", [False, True])
def test_reference_tree_buffers_linear_in_length(causal):
    """On the reference's tree (binary, one token per leaf) the sampler's deep
    levels run per sampled path and the backward's in bands, so the forward and
    backward workspaces grow linearly with L (the op-level problem at B=2, H=16,
    D=128, S=16), and so does the record: with more leaf blocks than the
    counting sort's window, pairs are bucketed by a radix sort with one count
    per leaf block instead of a (leaf block x query chunk) table."""
    from treeattention_amd import _lib

    sizes = {L: _lib.byte_sizes(_ref_tree_problem(L, causal)) for L in (4096, 16384, 65536)}
    for L in sizes:
        rec, fws, bws = sizes[L]
        print(L, rec / 2**30, fws / 2**30, bws / 2**30)
        assert fws == 0  # the leaf stage of one-token leaves is a value gather
    r16, r64 = sizes[16384][2], sizes[65536][2]
    assert r64 < 4.4 * r16  # linear (a dense child-logit gradient would be 16x)
    assert sizes[65536][2] < 24 * 2**30  # fits one GPU with room (was 565 GB)
    assert sizes[65536][0] < 4.4 * sizes[16384][0]
    assert sizes[65536][0] < 8 * 2**30


def test_bench_reads_committed_counter_summaries():
    """bench.py's roofline object takes its traffic and counter MFMA figures from the committed
    rocprofv3 summaries; every summary present must parse and hold plausible values."""
    import importlib.util

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location("bench", os.path.join(root, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    found = 0
    for cfg in bench.CONFIGS:
        if os.path.exists(os.path.join(root, "profiles", f"traffic_{cfg}.md")):
            t = bench.read_traffic("leaf_backward", cfg)
            assert t is not None and 1e6 < t < 1e11, (cfg, t)
            found += 1
        if os.path.exists(os.path.join(root, "profiles", f"mfma_{cfg}.md")):
            for ph in ("leaf_forward", "leaf_backward"):
                fr = bench.read_profile("mfma", "mfma_counter_frac", ph, cfg)
                ut = bench.read_profile("mfma", "mfma_util_pct", ph, cfg)
                if fr is None:  # one-token leaves: no MFMA leaf kernel
                    continue
                assert 0 < fr < 1 and 0 < ut < 100, (cfg, ph, fr, ut)
    assert found >= 1
    assert bench.read_profile("mfma", "mfma_util_pct", "leaf_backward", "no-such-config") is None
