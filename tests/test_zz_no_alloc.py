"""``ta_forward_static`` (the forward that allocates nothing: its pair rows live
in the library's static device scratch) against ``ta_forward`` through the C
ABI: out, weights and sampled leaves bit-identical, on two calls in a row, the
second with a smaller input; and its size limit."""

from __future__ import annotations

import ctypes

import pytest
import torch

TA_STATIC_SCRATCH_BYTES = 128 << 20


def _inputs(B, L, H, D, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [torch.randn(B, L, H, D, device="cuda", generator=g).to(dtype) for _ in range(3)]


def _static_forward(q, k, v, opts):
    from treeattention_amd import _lib
    from treeattention_amd.function import _strides, make_problem

    lib = _lib.load()
    prob = make_problem(q, k, v, opts)
    rec_b, _, _ = _lib.byte_sizes(prob)
    out = torch.empty_like(q)
    prob.o_strides[:] = _strides(out, opts.layout)
    w = torch.empty((*q.shape[:3], opts.num_samples), device=q.device, dtype=torch.float32)
    prob.w_strides[:] = _strides(w, opts.layout)
    rec = torch.empty(rec_b, device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        _lib.check(lib.ta_forward_static(ctypes.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(), None,
                                         ctypes.c_uint64(opts.seed), out.data_ptr(), w.data_ptr(), rec.data_ptr(),
                                         torch.cuda.current_stream(q.device).cuda_stream))
    return out, w, rec


@pytest.mark.gpu
def test_static_forward_matches_workspace_forward():
    from treeattention_amd.function import TreeOptions, record_views, tree_forward

    cases = [
        # several (batch, head) groups: 16 MiB of pair rows per (batch, head), 8 per group
        ((2, 4096, 8, 128, torch.bfloat16, 7), dict(num_samples=16, branching=4, leaf_block=64, tree_mode="natural",
                                                    causal=True, seed=3)),
        # then a smaller one (a single group) in float32
        ((1, 1024, 2, 64, torch.float32, 8), dict(num_samples=8, branching=2, leaf_block=16, tree_mode="compat",
                                                  causal=False, seed=5)),
    ]
    for (B, L, H, D, dtype, seed), kw in cases:
        print(f"[case] static forward B={B} L={L} H={H} D={D} {dtype} {kw}", flush=True)
        q, k, v = _inputs(B, L, H, D, dtype, seed)
        opts = TreeOptions(**kw)
        out_r, w_r, rec_r = tree_forward(q, k, v, opts)
        out_s, w_s, rec_s = _static_forward(q, k, v, opts)
        torch.cuda.synchronize()
        assert torch.equal(out_s, out_r)
        assert torch.equal(w_s, w_r)
        assert torch.equal(record_views(q, k, v, opts, rec_s)[0], record_views(q, k, v, opts, rec_r)[0])
        assert torch.isfinite(out_s.float()).all()


def test_static_forward_rejects_problems_over_its_scratch():
    """One (batch, head) of L * S * D * 2 bytes above the scratch: a clear error
    from the host-side checks, before anything touches a device."""
    from treeattention_amd import _lib

    lib = _lib.load()
    p = _lib.Problem()
    p.B, p.L, p.H, p.D, p.N = 1, 65536, 1, 128, 65536
    p.num_samples, p.branching, p.leaf_block = 16, 2, 128
    p.tree_mode, p.causal, p.dtype = _lib.TA_TREE_COMPAT, _lib.TA_CAUSAL_NONE, _lib.TA_BF16
    p.scale, p.max_logit = 0.1, 1e3
    for f in ("q_strides", "k_strides", "v_strides", "o_strides", "g_strides", "w_strides"):
        getattr(p, f)[:] = (65536 * 128, 128, 128)
    assert 65536 * 16 * 128 * 2 > TA_STATIC_SCRATCH_BYTES
    rc = lib.ta_forward_static(ctypes.byref(p), None, None, None, None, 0, None, None, None, None)
    assert rc == _lib.TA_ERR_UNSUPPORTED
    assert "static scratch" in lib.ta_last_error().decode()
