"""GPU tests of more than 64 samples per query (the reference only asks
``num_samples > 0``, ``_autograd.py:657-658``, default 64 at ``_tree_mha.py:331``).

The library draws and uses the samples in chunks of at most 64 and joins the
chunks by their log-normalizers; every result must equal the one softmax over
all samples that the reference takes (``_tree_mha.py:396-407``):

* leaves bit-exact against the oracle's sampling with the same uniforms where
  every decision's margin exceeds 1e-3 (the chunks index the uniforms of their
  global sample numbers), weights, output and gradients against the oracle on
  the GPU's paths at 1e-5 (float32) / 2e-2 (16-bit) -- ``run_case``;
* the in-kernel counter RNG equals explicit uniforms, runs are bitwise
  reproducible, and a forward's own paths replay bit for bit;
* the op-level API against the reference-structure restatement;
* the reference causal mode, which couples every sample of a query in one
  workgroup, refuses more than 64 with a clear error.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import treeattention_amd as ta
from oracle import tree_oracle as O
from tests.test_gpu_parity import f64, make_inputs, rel, run_case
from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,b,LB,L,D,causal,dtype", [
    (100, 2, 16, 256, 64, False, torch.float32),    # two chunks of 50
    (130, 4, 16, 256, 64, True, torch.bfloat16),    # three chunks, exact causal
    (65, 2, 64, 1024, 128, True, torch.float16),    # 33 + 32, the C3-size leaf tiles
    (256, 4, 64, 1024, 32, False, torch.bfloat16),  # four full chunks
])
def test_many_samples_against_oracle(S, b, LB, L, D, causal, dtype):
    run_case(1, L, 2, D, S, b, LB, "natural", causal, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_many_samples_reference_tree(dtype):
    # one token per leaf (the value gather), compat summaries, non-causal
    run_case(2, 64, 2, 32, 96, 2, 1, "compat", False, dtype)


def test_many_samples_sparse_levels():
    # per-path sampler levels and node-major bands forced on, chunks of 40
    run_case(1, 512, 2, 32, 80, 2, 1, "compat", False, torch.bfloat16, dense_cols=32)
    run_case(1, 1024, 2, 64, 72, 2, 4, "natural", True, torch.float32, dense_cols=32)


def test_many_samples_seed_path_replay_and_determinism():
    B, L, H, D, S, b, LB = 1, 512, 2, 64, 100, 4, 32
    print(f"[case] seed / replay S={S}", flush=True)
    q, k, v, do = (x.cuda() for x in make_inputs(B, L, H, D, torch.bfloat16, 5))
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode="natural", causal=False, seed=9)
    T = O.tree_depth(L // LB, b)
    U = torch.from_numpy(O.uniforms(9, (B, L, H, S, T, b))).cuda()
    o1, w1, r1 = tree_forward(q, k, v, opts)
    o2, w2, _ = tree_forward(q, k, v, opts, U)
    o3, w3, r3 = tree_forward(q, k, v, opts)
    assert torch.equal(o1, o2) and torch.equal(w1, w2) and torch.equal(o1, o3) and torch.equal(w1, w3)
    torch.testing.assert_close(w1.sum(-1), torch.ones_like(w1[..., 0]), rtol=0, atol=1e-5)
    g1 = tree_backward(q, k, v, w1, r1, do, opts)
    g3 = tree_backward(q, k, v, w3, r3, do, opts)
    for a, c in zip(g1, g3):
        assert torch.equal(a, c)
    # the forward's own paths, packed and replayed, reproduce it
    leaves = record_views(q, k, v, opts, r1)[0]
    paths = ta.pack_paths(leaves, L // LB, layout="blhs")
    o4, w4, r4 = tree_forward(q, k, v, opts, paths=paths)
    assert torch.equal(o1, o4) and torch.equal(w1, w4)
    for a, c in zip(g1, tree_backward(q, k, v, w4, r4, do, opts)):
        assert torch.equal(a, c)


def test_many_samples_op_level():
    """hierarchical_attention with num_samples = 128 (non-causal, node keys) against the
    reference-structure restatement on the GPU's paths."""
    L, B, H, D, S = 64, 2, 2, 32, 128
    print(f"[case] op-level S={S}", flush=True)
    E = H * D
    g = torch.Generator().manual_seed(4321)
    query, value, gout = (torch.randn(L, B, E, generator=g) for _ in range(3))
    key = torch.randn(L - 1, B, E, generator=g)
    T = int(math.log2(L))
    U = O.uniforms(0, (B, L, H, S, T, 2))
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (query, key, value))
    out, w, paths = ta.hierarchical_attention(qd, kd, vd, num_heads=H, num_samples=S,
                                              uniforms=torch.from_numpy(U).cuda(), return_paths=True)
    out.backward(gout.cuda())
    q4, v4 = (x.double().numpy().reshape(L, B, H, D).transpose(1, 0, 2, 3) for x in (query, value))
    k4 = key.double().numpy().reshape(L - 1, B, H, D)
    C = O.nodekeys_to_summaries(k4.transpose(1, 2, 0, 3))
    _, _, margins = O.tree_sample(q4, C, 2, 1, U, False)
    idx_o = O.tree_sample(q4, C, 2, 1, U, False)[0]
    leaves = O.unpack_paths(paths.cpu().numpy(), L).transpose(1, 0, 2, 3)
    clean = margins.min(axis=-1) > 1e-3
    assert not ((leaves != idx_o) & clean).any()
    wb = O.sample_weights(O.path_logprobs(q4, C, 2, L, leaves))
    o_s, _ = O.leaf_attention(q4, np.zeros_like(v4), v4, leaves, 1, False, 1.0)
    out_ref = np.einsum("blhs,blhsd->blhd", wb, o_s)
    assert rel(f64(out), out_ref.transpose(1, 0, 2, 3).reshape(L, B, E)) < 1e-5
    assert rel(w.detach().cpu().numpy(), wb.transpose(1, 0, 2, 3)) < 1e-5
    dq, dC, _, dv = O.tree_backward(q4, np.zeros_like(v4), v4, C, 2, 1, leaves, wb,
                                    gout.double().numpy().reshape(L, B, H, D).transpose(1, 0, 2, 3), False)
    assert rel(f64(qd.grad).reshape(L, B, H, D).transpose(1, 0, 2, 3), dq) < 1e-5
    assert rel(f64(kd.grad).reshape(L - 1, B, H, D).transpose(1, 2, 0, 3), O.nodekeys_adjoint(dC)) < 1e-5
    assert rel(f64(vd.grad).reshape(L, B, H, D).transpose(1, 0, 2, 3), dv) < 1e-5


def test_many_samples_reference_causal_is_refused():
    L, B, H, D = 64, 1, 2, 32
    q = torch.randn(L, B, H * D, device="cuda:0")
    k = torch.randn(L - 1, B, H * D, device="cuda:0")
    v = torch.randn(L, B, H * D, device="cuda:0")
    with pytest.raises(RuntimeError, match="couples every sample"):
        ta.hierarchical_attention(q, k, v, num_heads=H, is_causal=True, num_samples=65)
