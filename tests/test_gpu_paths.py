"""GPU tests of the packed path record and path replay.

* ``pack_paths`` / ``unpack_paths`` kernels against the oracle (pinned by the
  reference's heap walk in ``tests/test_paths.py``), 0 to 4 bytes per path,
  both leaf layouts.
* Replaying the reference's own sampled paths (the ``idx`` of the non-causal
  golden fixtures, written by ``treeattn_torch``) through the op reproduces the
  reference's outputs, weights and gradients -- independent of the noise
  stream that drew them.
* Replaying a forward's own paths (``return_paths=True``) reproduces it bit for
  bit, on the reference tree and on a generalized tree (b = 4, LB = 64).
* Replay of given (unsampled) leaf blocks on a generalized tree against the
  oracle's path log-probabilities, weights, output and gradients.

Bar: bit-exact for ids and bytes and for self-replay; 1e-5 (float32) / 2e-2
(bfloat16) norm-wise relative error against the reference and the oracle.
"""

from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest
import torch

import treeattention_amd as ta
from oracle import tree_oracle as O
from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
DEV = torch.device("cuda:0")
NONCAUSAL = sorted(glob.glob(os.path.join(HERE, "golden", "noncausal_*.npz")))


def rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("nl", [1, 2, 256, 512, 1 << 17, 1 << 24, 1 << 30])
def test_pack_unpack_kernels_match_oracle(nl):
    print(f"[case] pack/unpack NL={nl}", flush=True)
    rng = np.random.default_rng(nl % 1000)
    leaf = rng.integers(0, nl, size=(37, 2, 3, 5)).astype(np.int32)  # (L, B, H, S)
    lg = torch.as_tensor(leaf).to(DEV)
    packed = ta.pack_paths(lg, nl)  # reference layout input
    ref = O.pack_paths(leaf, nl)
    assert packed.shape == ref.shape and packed.dtype == torch.uint8
    np.testing.assert_array_equal(packed.cpu().numpy(), ref)
    # the record's (B, L, H, S) layout, and a strided view, give the same bytes
    blhs = lg.permute(1, 0, 2, 3).contiguous()
    np.testing.assert_array_equal(ta.pack_paths(blhs, nl, layout="blhs").cpu().numpy(), ref)
    np.testing.assert_array_equal(ta.pack_paths(blhs.permute(1, 0, 2, 3), nl).cpu().numpy(), ref)
    back = ta.unpack_paths(packed, nl)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back.cpu().numpy(), leaf if nl > 1 else np.zeros_like(leaf))


def test_pack_empty_and_bad_arguments():
    e = torch.zeros((0, 2, 3, 4), dtype=torch.int32, device=DEV)
    assert ta.pack_paths(e, 256).shape == (0, 2, 3, 4, 1)
    with pytest.raises(ValueError):
        ta.pack_paths(e.float(), 256)
    with pytest.raises(ValueError):
        ta.pack_paths(e, 12)  # not a power of two
    with pytest.raises(ValueError):
        ta.unpack_paths(torch.zeros((1, 1, 1, 1, 2), dtype=torch.uint8, device=DEV), 256)  # wrong byte count


@pytest.mark.parametrize("path", NONCAUSAL, ids=[os.path.basename(p)[:-4] for p in NONCAUSAL])
def test_replaying_reference_paths_reproduces_reference(path):
    z = np.load(path, allow_pickle=False)
    fx = {k: z[k] for k in z.files}
    L, B, H, D, S = (int(fx[k]) for k in ("L", "B", "H", "D", "S"))
    bf16 = str(fx["dtype"]) == "bfloat16"
    dtype = torch.bfloat16 if bf16 else torch.float32
    tol = 2e-2 if bf16 else 1e-5
    print(f"[case] replay fixture {os.path.basename(path)}", flush=True)
    N = L
    packed = ta.pack_paths(torch.as_tensor(fx["idx"].astype(np.int32)).to(DEV), N)
    np.testing.assert_array_equal(packed.cpu().numpy(), O.pack_paths(fx["idx"], N))
    q, k, v = (torch.as_tensor(fx[n]).reshape(fx[n].shape[0], B, H * D).to(dtype).to(DEV).requires_grad_(True)
               for n in ("q", "k", "v"))
    out, w = ta.hierarchical_attention(q, k, v, num_heads=H, num_samples=S, paths=packed)
    out.backward(torch.as_tensor(fx["dout"]).to(dtype).to(DEV))
    torch.cuda.synchronize()
    for nm, got in (("out", f64(out)), ("weights", f64(w)), ("dq", f64(q.grad)), ("dk", f64(k.grad)),
                    ("dv", f64(v.grad))):
        assert rel(got, fx[nm]) < tol, (nm, rel(got, fx[nm]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_self_replay_reference_tree_is_bitwise(dtype):
    L, B, H, D, S = 256, 2, 2, 64, 8
    print(f"[case] self replay reference tree {dtype}", flush=True)
    g = torch.Generator().manual_seed(5)
    q, v, dout = (torch.randn(L, B, H * D, generator=g).to(dtype).to(DEV) for _ in range(3))
    k = (torch.randn(L - 1, B, H * D, generator=g) / 8).to(dtype).to(DEV)
    res = []
    for paths in (None, "replay"):
        qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
        if paths is None:
            out, w, packed = ta.hierarchical_attention(qg, kg, vg, num_heads=H, num_samples=S, seed=3,
                                                       return_paths=True)
            assert packed.shape == (L, B, H, S, 1) and packed.dtype == torch.uint8
        else:
            out, w = ta.hierarchical_attention(qg, kg, vg, num_heads=H, num_samples=S, seed=99, paths=packed)
        out.backward(dout)
        res.append((out.detach(), w, qg.grad, kg.grad, vg.grad))
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)


def _bshd(B, L, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, L, H, D, generator=g).to(dtype).to(DEV) for _ in range(4)]


def test_self_replay_generalized_tree_is_bitwise():
    B, L, H, D, S = 1, 4096, 4, 128, 16
    print("[case] self replay b=4 LB=64 natural", flush=True)
    q, k, v, dout = _bshd(B, L, H, D, torch.bfloat16, 7)
    opts = TreeOptions(num_samples=S, branching=4, leaf_block=64, tree_mode="natural", causal=False, seed=11,
                       layout="bshd")
    out1, w1, rec1 = tree_forward(q, k, v, opts)
    leaves = record_views(q, k, v, opts, rec1)[0]
    packed = ta.pack_paths(leaves, L // 64, layout="blhs")
    assert packed.shape == (L, B, H, S, 1)
    out2, w2, rec2 = tree_forward(q, k, v, opts, paths=packed)
    g1 = tree_backward(q, k, v, w1, rec1, dout, opts)
    g2 = tree_backward(q, k, v, w2, rec2, dout, opts)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2) and torch.equal(w1, w2)
    assert torch.equal(record_views(q, k, v, opts, rec2)[0], leaves)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("b,LB,mode", [(4, 64, "natural"), (2, 32, "compat")])
def test_replay_given_leaves_matches_oracle(b, LB, mode):
    B, L, H, D, S = 1, 1024, 2, 64, 8
    print(f"[case] replay given leaves b={b} LB={LB} {mode}", flush=True)
    q, k, v, dout = _bshd(B, L, H, D, torch.bfloat16, 13)
    nl = L // LB
    rng = np.random.default_rng(b)
    idx = rng.integers(0, nl, size=(B, L, H, S))
    packed = ta.pack_paths(torch.as_tensor(idx.astype(np.int32)).to(DEV), nl, layout="blhs")
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out, w = ta.tree_attention(qg, kg, vg, False, None, num_samples=S, branching=b, leaf_block=LB, tree_mode=mode,
                               paths=packed, return_weights=True)
    out.backward(dout)
    torch.cuda.synchronize()
    q64, k64, v64, d64 = (x.double().cpu().numpy() for x in (q, k, v, dout))
    C = O.summaries(k64, b, LB, mode)
    lp = O.path_logprobs(q64, C, b, nl, idx)
    w_ref = O.sample_weights(lp)
    o_s, _ = O.leaf_attention(q64, k64, v64, idx, LB, False, 1.0 / math.sqrt(D))
    out_ref = np.einsum("blhs,blhsd->blhd", w_ref, o_s)
    dq, dC, dk_leaf, dv = O.tree_backward(q64, k64, v64, C, b, LB, idx, w_ref, d64, False)
    dk = dk_leaf + O.pool_adjoint(dC, L, b, LB, mode)
    assert rel(f64(w), w_ref) < 1e-4
    assert rel(f64(out), out_ref) < 2e-2
    for got, ref in ((qg.grad, dq), (kg.grad, dk), (vg.grad, dv)):
        assert rel(f64(got), ref) < 2e-2


def test_replay_is_refused_for_causal_and_bad_shapes():
    L, B, H, D = 64, 1, 2, 32
    x = torch.randn(L, B, H * D, device=DEV)
    packed = torch.zeros((L, B, H, 4, 1), dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError):
        ta.hierarchical_attention(x, x[:-1], x, num_heads=H, is_causal=True, num_samples=4, paths=packed)
    with pytest.raises(ValueError):
        ta.hierarchical_attention(x, x[:-1], x, num_heads=H, num_samples=8, paths=packed)  # S mismatch
    with pytest.raises(ValueError):
        ta.hierarchical_attention(x, x[:-1], x, num_heads=H, mode="deterministic", paths=packed)
