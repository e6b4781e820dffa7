"""Pins the timed CPU baseline (``oracle/cpu_path.py``, float32 torch, the
reference's op order) against the float64 oracle: summaries and their adjoint,
sampled leaf blocks, weights, output and gradients on the same paths."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import cpu_path as P
from oracle import tree_oracle as O


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("b,LB,mode", [(2, 1, "compat"), (2, 4, "compat"), (4, 2, "natural"), (2, 3, "natural")])
def test_summaries_and_adjoint(b, LB, mode):
    rng = np.random.default_rng(1)
    H, D = 3, 5
    N = LB * b**3
    k = rng.standard_normal((1, N, H, D))
    C = P.summaries(torch.tensor(k, dtype=torch.float32)[0], b, LB, mode)
    np.testing.assert_allclose(C.numpy(), O.summaries(k, b, LB, mode)[0], rtol=1e-5, atol=1e-6)
    dC = rng.standard_normal((1, H, C.shape[1], D))
    ref = O.pool_adjoint(dC, N, b, LB, mode)[0]
    got = P.summaries_adjoint(torch.tensor(dC[0], dtype=torch.float32), N, b, LB, mode)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("b,LB,causal,mode,NmL", [
    (2, 1, False, "compat", 0), (4, 4, True, "natural", 0), (2, 4, True, "compat", 8), (4, 2, False, "natural", 0),
])
def test_forward_backward_match_oracle(b, LB, causal, mode, NmL):
    rng = np.random.default_rng(2)
    H, D, S = 2, 8, 5
    T = 3
    N = LB * b**T
    L = N - NmL
    q, g = (rng.standard_normal((1, L, H, D)).astype(np.float32) for _ in range(2))
    k, v = (rng.standard_normal((1, N, H, D)).astype(np.float32) for _ in range(2))
    U = O.uniforms(3, (1, L, H, S, T, b))
    C64 = O.summaries(k.astype(np.float64), b, LB, mode)
    idx_o, _, margins = O.tree_sample(q, C64, b, LB, U, causal, N=N)
    prob = P.Problem(torch.tensor(q[0]), torch.tensor(k[0]), torch.tensor(v[0]), torch.tensor(U[0]),
                     torch.arange(L) + (N - L), b, LB, causal, mode, scale=0.3, qblock=7)
    C = P.summaries(prob.k, b, LB, mode)
    idx, w, out = prob.forward(C)
    clean = margins.min(-1)[0] > 1e-3
    assert clean.mean() > 0.9
    np.testing.assert_array_equal(idx.numpy()[clean], idx_o[0][clean])
    # everything else on the oracle's paths
    idx, w, out = prob.forward(C, forced=torch.tensor(idx_o[0]))
    np.testing.assert_array_equal(idx.numpy(), idx_o[0])
    res = O.attention_fwd_bwd(q, k, v, g, b, LB, U, causal, mode, scale=0.3)
    w_ref = O.sample_weights(O.path_logprobs(q, C64, b, N // LB, idx_o))
    o_s, _ = O.leaf_attention(q, k, v, idx_o, LB, causal, 0.3)
    out_ref = np.einsum("blhs,blhsd->blhd", w_ref, o_s)
    assert rel(w.numpy(), w_ref[0]) < 1e-5 and rel(out.numpy(), out_ref[0]) < 1e-5
    dq_o, dC, dkl, dv_o = O.tree_backward(q, k, v, C64, b, LB, idx_o, w_ref, g, causal, 0.3)
    dk_o = dkl + O.pool_adjoint(dC, N, b, LB, mode)
    dq, dk, dv = prob.backward(C, idx, w, torch.tensor(g[0]))
    for got, ref in ((dq, dq_o), (dk, dk_o), (dv, dv_o)):
        assert rel(got.numpy(), ref[0]) < 1e-5
    if NmL == 0 and not causal:
        np.testing.assert_allclose(out.numpy(), res["out"][0], rtol=1e-4, atol=1e-5)
