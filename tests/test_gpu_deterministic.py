"""GPU parity of the deterministic (exact) mode (``_tree_mha.py:271-321``).

* Against the reference itself: ``tests/golden/deterministic_{noncausal,causal}_f32_L16.npz``
  hold the outputs, weights and autograd gradients of
  ``treeattn_torch.hierarchical_attention(..., mode="deterministic")``.
* Against the float64 restatement ``oracle/ref_torch.deterministic_attention``
  (pinned by those fixtures in ``tests/test_golden.py``) with autograd for the
  gradients, at larger sizes, in float32 / bfloat16 / float16, causal or not,
  with ``L != N``.
* The attn-bench adapter's deterministic path (``TREEATTN_NUM_SAMPLES`` unset,
  ``baselines/treeattn_torch.py:48-90``): Haar node keys of ``k`` (oracle
  ``haar_inorder``, read in heap order) and ``dk`` through the Haar adjoint.

Bar: 1e-5 (float32) / 2e-2 (16-bit) norm-wise relative error.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import treeattention_amd as ta
from oracle import ref_torch as R
from oracle import tree_oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f64(t) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def run_op(q, k, v, dout, H, causal, dtype):
    """GPU op-level call on (L,B,E) tensors: (out, weights, dq, dk, dv) as float64 arrays."""
    qg, kg, vg = (torch.as_tensor(x).to(dtype).to(DEV).requires_grad_(True) for x in (q, k, v))
    out, w = ta.hierarchical_attention(qg, kg, vg, num_heads=H, is_causal=causal, mode="deterministic")
    out.backward(torch.as_tensor(dout).to(dtype).to(DEV))
    torch.cuda.synchronize()
    return f64(out), f64(w), f64(qg.grad), f64(kg.grad), f64(vg.grad)


@pytest.mark.parametrize("name", ["deterministic_noncausal_f32_L16", "deterministic_causal_f32_L16"])
def test_matches_reference_fixture(name):
    z = np.load(os.path.join(HERE, "golden", name + ".npz"))
    L, B, H, D = z["q"].shape
    causal = bool(z["causal"])
    print(f"[case] fixture {name} L={L} B={B} H={H} D={D} causal={causal}", flush=True)
    q, k, v = (z[n].reshape(z[n].shape[0], B, H * D) for n in ("q", "k", "v"))
    out, w, dq, dk, dv = run_op(q, k, v, z["dout"], H, causal, torch.float32)
    assert w.shape == z["weights"].shape
    for nm, got in (("out", out), ("weights", w), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert rel(got, z[nm]) < 1e-5, (nm, rel(got, z[nm]))


def _oracle(q, k, v, dout, causal):
    """float64 restatement with autograd: (out (L,B,H,D), w, dq, dk, dv)."""
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    out, w = R.deterministic_attention(qt, kt, vt, causal)
    out.backward(torch.tensor(dout, dtype=torch.float64))
    return out.detach().numpy(), w.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


CASES = [
    # L, N, B, H, D, dtype, causal
    (256, 256, 2, 2, 64, torch.float32, False),
    (256, 256, 2, 2, 64, torch.float32, True),
    (96, 128, 1, 3, 32, torch.float32, True),
    (160, 128, 1, 2, 32, torch.float32, False),
    (512, 512, 1, 2, 128, torch.bfloat16, True),
    (256, 256, 2, 2, 96, torch.bfloat16, False),
    (256, 256, 1, 4, 64, torch.float16, True),
]


@pytest.mark.parametrize("L,N,B,H,D,dtype,causal", CASES)
def test_against_restatement(L, N, B, H, D, dtype, causal):
    print(f"[case] L={L} N={N} B={B} H={H} D={D} {dtype} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(L + N + D)
    q = torch.randn(L, B, H, D, generator=g).to(dtype)
    k = (torch.randn(N - 1, B, H, D, generator=g) / D ** 0.5).to(dtype)
    v = torch.randn(N, B, H, D, generator=g).to(dtype)
    dout = torch.randn(L, B, H, D, generator=g).to(dtype)
    ref = _oracle(*(x.double().numpy() for x in (q, k, v, dout)), causal)
    got = run_op(q.reshape(L, B, H * D), k.reshape(N - 1, B, H * D), v.reshape(N, B, H * D),
                 dout.reshape(L, B, H * D), H, causal, dtype)
    shapes = [(L, B, H, D), (L, B, H, N), (L, B, H, D), (N - 1, B, H, D), (N, B, H, D)]
    for nm, a, r, sh in zip(("out", "weights", "dq", "dk", "dv"), got, ref, shapes):
        a = a.reshape(sh)
        assert rel(a, r) < TOL[dtype], (nm, rel(a, r))
    if not causal:
        assert np.allclose(got[1].sum(-1), 1.0, atol=1e-4)  # exact path probabilities sum to one


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adapter_deterministic_path(monkeypatch, causal, dtype):
    monkeypatch.delenv("TREEATTN_NUM_SAMPLES", raising=False)
    for var in ("TREEATTN_BRANCHING", "TREEATTN_LEAF_BLOCK", "TREEATTN_TREE_MODE"):
        monkeypatch.delenv(var, raising=False)
    B, S, H, D = 2, 128, 2, 32
    print(f"[case] adapter deterministic B={B} S={S} H={H} D={D} {dtype} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(7)
    q, k, v, dout = (torch.randn(B, S, H, D, generator=g).to(dtype) for _ in range(4))
    qg, kg, vg = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out = ta.attn_fn(qg, kg, vg, causal, None)
    assert out.shape == q.shape and out.dtype == dtype
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    # oracle: Haar node keys (in-order coefficients, read in heap order) of the sbhd keys
    q64, k64, v64, d64 = (x.double().numpy().transpose(1, 0, 2, 3) for x in (q, k, v, dout))
    knode = O.haar_inorder(k64)  # (S-1, B, H, D)
    out_r, _, dq_r, dkn_r, dv_r = _oracle(q64, knode, v64, d64, causal)
    dk_r = O.haar_inorder_adjoint(dkn_r)
    tol = TOL[dtype]
    tr = lambda a: a.transpose(1, 0, 2, 3)  # noqa: E731
    assert rel(f64(out), tr(out_r)) < tol
    assert rel(f64(qg.grad), tr(dq_r)) < tol
    assert rel(f64(kg.grad), tr(dk_r)) < tol
    assert rel(f64(vg.grad), tr(dv_r)) < tol


def test_haar_node_keys_match_oracle():
    from treeattention_amd.function import haar_node_keys, haar_node_keys_adjoint

    B, S, H, D = 2, 256, 3, 64
    g = torch.Generator().manual_seed(3)
    k = torch.randn(B, S, H, D, generator=g)
    kt = haar_node_keys(k.to(DEV))
    ref = O.haar_inorder(k.double().numpy().transpose(1, 0, 2, 3))
    assert rel(f64(kt), ref) < 1e-6
    dkey = torch.randn(S - 1, B, H, D, generator=g)
    dk = haar_node_keys_adjoint(dkey.to(DEV), k.to(DEV))
    ref_adj = O.haar_inorder_adjoint(dkey.double().numpy()).transpose(1, 0, 2, 3)
    assert rel(f64(dk), ref_adj) < 1e-6


def test_edge_cases_and_limits():
    B, H, D = 1, 2, 32
    x = torch.randn(5, B, H * D, device=DEV)
    v1 = torch.randn(1, B, H * D, device=DEV)
    out, w = ta.hierarchical_attention(x, x[:0], v1, num_heads=H, mode="deterministic")
    assert torch.equal(out, v1.expand(5, -1, -1)) and w.shape == (5, B, H, 1)
    out0, w0 = ta.hierarchical_attention(x, x[:0], x[:0], num_heads=H, mode="deterministic")
    assert torch.equal(out0, torch.zeros_like(x)) and w0.shape == (5, B, H, 0)
    with pytest.raises(NotImplementedError):  # N must be a power of two
        ta.hierarchical_attention(x, x[:5], torch.randn(6, B, H * D, device=DEV), num_heads=H, mode="deterministic")


def test_deterministic_mode_is_bitwise_reproducible():
    L, B, H, D = 128, 1, 2, 64
    g = torch.Generator().manual_seed(11)
    q, v = (torch.randn(L, B, H * D, generator=g).to(DEV) for _ in range(2))
    k = torch.randn(L - 1, B, H * D, generator=g).to(DEV) / 8
    o1, w1 = ta.hierarchical_attention(q, k, v, num_heads=H, is_causal=True, mode="deterministic")
    o2, w2 = ta.hierarchical_attention(q, k, v, num_heads=H, is_causal=True, mode="deterministic")
    assert torch.equal(o1, o2) and torch.equal(w1, w2)


STREAM_CASES = [
    # N (= L), D, dtype, causal
    (64, 64, torch.bfloat16, False),
    (64, 32, torch.float16, True),
    (256, 128, torch.bfloat16, True),
    (1024, 96, torch.float16, False),
    (1024, 64, torch.bfloat16, True),
    (4096, 128, torch.bfloat16, False),
]


@pytest.mark.parametrize("N,D,dtype,causal", STREAM_CASES)
def test_streaming_forward_matches_restatement(N, D, dtype, causal):
    """The streaming forward (no (L, N) weights) against the float64 restatement, with the node keys
    rounded to the input type as the kernel reads them."""
    from treeattention_amd.function import det_stream_forward

    B, H = 1, 2
    print(f"[case] stream fwd N={N} D={D} {dtype} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(N + D)
    q = torch.randn(B, N, H, D, generator=g).to(dtype)
    kn = (torch.randn(N - 1, B, H, D, generator=g) / D ** 0.5).to(dtype)
    v = torch.randn(B, N, H, D, generator=g).to(dtype)
    out = det_stream_forward(q.to(DEV), kn.to(DEV), v.to(DEV), causal)
    torch.cuda.synchronize()
    qt, kt, vt = (torch.tensor(x.double().numpy()) for x in (q.permute(1, 0, 2, 3), kn, v.permute(1, 0, 2, 3)))
    ref, _ = R.deterministic_attention(qt, kt, vt, causal)
    assert out.shape == q.shape and out.dtype == dtype
    assert rel(f64(out).transpose(1, 0, 2, 3), ref.numpy()) < 2e-2


def test_streaming_adapter_path_long_causal(monkeypatch):
    """Adapter deterministic path at S = 2048 (streaming forward, recomputed backward) against the
    float64 restatement with the oracle's Haar node keys."""
    monkeypatch.delenv("TREEATTN_NUM_SAMPLES", raising=False)
    for var in ("TREEATTN_BRANCHING", "TREEATTN_LEAF_BLOCK", "TREEATTN_TREE_MODE"):
        monkeypatch.delenv(var, raising=False)
    B, S, H, D = 1, 2048, 2, 64
    print(f"[case] adapter deterministic streaming S={S}", flush=True)
    g = torch.Generator().manual_seed(17)
    q, k, v, dout = (torch.randn(B, S, H, D, generator=g).to(torch.bfloat16) for _ in range(4))
    qg, kg, vg = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    out = ta.attn_fn(qg, kg, vg, True, None)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    q64, k64, v64, d64 = (x.double().numpy().transpose(1, 0, 2, 3) for x in (q, k, v, dout))
    out_r, _, dq_r, dkn_r, dv_r = _oracle(q64, O.haar_inorder(k64), v64, d64, True)
    tr = lambda a: a.transpose(1, 0, 2, 3)  # noqa: E731
    assert rel(f64(out), tr(out_r)) < 2e-2
    assert rel(f64(qg.grad), tr(dq_r)) < 2e-2
    assert rel(f64(kg.grad), tr(O.haar_inorder_adjoint(dkn_r))) < 2e-2
    assert rel(f64(vg.grad), tr(dv_r)) < 2e-2


@pytest.mark.parametrize("N,D,dtype,causal", STREAM_CASES + [(128, 64, torch.bfloat16, True)])
def test_streaming_backward_matches_restatement(N, D, dtype, causal):
    """The streaming backward (subtree kernels + coarse top tree) against float64 autograd of the
    restatement, node keys rounded to the input type as the kernels read them."""
    from treeattention_amd.function import det_stream_backward, det_stream_forward

    B, H = 1, 2
    print(f"[case] stream bwd N={N} D={D} {dtype} causal={causal}", flush=True)
    g = torch.Generator().manual_seed(3 * N + D)
    q = torch.randn(B, N, H, D, generator=g).to(dtype)
    kn = (torch.randn(N - 1, B, H, D, generator=g) / D ** 0.5).to(dtype)
    v, dout = (torch.randn(B, N, H, D, generator=g).to(dtype) for _ in range(2))
    qg, kg, vg, dg = (x.to(DEV) for x in (q, kn, v, dout))
    out, lse = det_stream_forward(qg, kg, vg, causal, return_lse=True)
    dq, dkn, dv = det_stream_backward(qg, kg, vg, dg, out, lse, causal)
    torch.cuda.synchronize()
    lbhd = lambda t: t.permute(1, 0, 2, 3)  # noqa: E731
    out_r, _, dq_r, dk_r, dv_r = _oracle(*(x.double().numpy() for x in (lbhd(q), kn, lbhd(v), lbhd(dout))), causal)
    assert rel(f64(lbhd(dq)), dq_r) < 2e-2, rel(f64(lbhd(dq)), dq_r)
    assert rel(f64(dkn), dk_r) < 2e-2, rel(f64(dkn), dk_r)
    assert rel(f64(lbhd(dv)), dv_r) < 2e-2, rel(f64(lbhd(dv)), dv_r)


@pytest.mark.parametrize("N,D,dtype", [(2, 32, torch.float32), (64, 96, torch.bfloat16), (128, 64, torch.float32),
                                       (4096, 128, torch.float32), (8192, 36, torch.float16)])
def test_haar_pyramid_matches_oracle(N, D, dtype):
    """The block-sum pyramid (segment levels in LDS, then the levels over segment sums) against the
    oracle's in-order Haar transform read in heap order."""
    from treeattention_amd.function import haar_node_keys

    B, H = 1, 2
    print(f"[case] haar pyramid N={N} D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(N + D)
    k = torch.randn(B, N, H, D, generator=g).to(dtype)
    kt = haar_node_keys(k.to(DEV))
    torch.cuda.synchronize()
    ref = O.haar_inorder(k.double().numpy().transpose(1, 0, 2, 3))
    assert rel(f64(kt), ref) < 1e-6
