"""The oracle's restatement of the reference op against the reference's own outputs.

The fixtures in ``tests/golden/`` were written by ``tests/golden/make_golden.py``,
which ran the reference implementation (``treeattn_torch._tree_mha``) with its
Gumbel noise taken from the same uniform tensor ``U`` stored in each fixture.
These tests pin ``oracle/ref_torch.py`` -- the non-causal sampler, the causal
two-pass sampler with its cross-lane coupling, the causal hybrid and the
deterministic mode -- including the gradients that autograd gives through it.

Bar: sampled indices identical wherever every decision margin exceeds 1e-3
(float32 fixtures) / 0.05 (bfloat16 fixtures, where the reference rounds its
dots, log-sigmoids and noise to bfloat16); outputs, weights and gradients within
1e-5 (float32) / 2e-2 (bfloat16) norm-wise relative error.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import ref_torch as R

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def load(path):
    z = np.load(path, allow_pickle=False)
    return {k: z[k] for k in z.files}


def run_oracle(fx, forced=None):
    L, B, H, D, S = (int(fx[k]) for k in ("L", "B", "H", "D", "S"))
    mode = str(fx["mode"])
    q, k, v = (torch.tensor(fx[n], dtype=torch.float64, requires_grad=True) for n in ("q", "k", "v"))
    out, w, info = R.hierarchical_attention(q.reshape(L, B, H * D), k.reshape(k.shape[0], B, H * D),
                                            v.reshape(v.shape[0], B, H * D), H, bool(fx["causal"]), mode, S,
                                            fx["U"], forced=forced)
    out.backward(torch.tensor(fx["dout"], dtype=torch.float64))
    return out.detach().numpy(), w.detach().numpy(), info, (q.grad.numpy(), k.grad.numpy(), v.grad.numpy())


def test_fixtures_present():
    names = {os.path.basename(p)[:-4] for p in FIXTURES}
    for need in ("noncausal_f32_L16", "causal_hybrid_f32_L32", "causal_short_f32_L8",
                 "deterministic_causal_f32_L16"):
        assert need in names


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_oracle_matches_reference_fixture(path):
    fx = load(path)
    bf16 = str(fx["dtype"]) == "bfloat16"
    tol = 2e-2 if bf16 else 1e-5
    out, w, info, (dq, dk, dv) = run_oracle(fx)
    if "idx" in fx:
        idx = info["idx"].numpy()
        clean = info["margins"].numpy().min(axis=-1) > (5e-2 if bf16 else 1e-3)
        assert clean.mean() > 0.9
        np.testing.assert_array_equal(idx[clean], fx["idx"][clean])
        # a near-tie may go either way between float64 and the reference's bfloat16
        # arithmetic; then the values are compared on the reference's own paths
        if not (idx == fx["idx"]).all():
            assert bf16, "float32 fixture: a near-tie decision flipped"
            out, w, info, (dq, dk, dv) = run_oracle(fx, forced=fx["idx"])
            np.testing.assert_array_equal(info["idx"].numpy(), fx["idx"])
    assert rel(out, fx["out"]) < tol
    assert w.shape == fx["weights"].shape
    assert rel(w, fx["weights"]) < tol
    for got, ref in ((dq, fx["dq"]), (dk, fx["dk"]), (dv, fx["dv"])):
        assert rel(got.reshape(ref.shape), ref) < tol


def test_causal_coupling_stops_correction_and_reaches_future_leaves():
    """The reference corrects only while every lane is on the boundary path; after that,
    samples may land right of the query (``_tree_mha.py:204-207``).  The fixtures hold
    both situations; the oracle reproduces them."""
    fx = load(os.path.join(HERE, "golden", "causal_hybrid_f32_L64.npz"))
    S = int(fx["S"])
    _, _, info, _ = run_oracle(fx)
    dstar = info["dstar"]
    T = (int(fx["L"]) - 1).bit_length()
    assert (dstar < T).any()
    t = np.arange(S, int(fx["L"]))[:, None, None, None]
    assert (fx["idx"] > t).any(), "no future leaf sampled in this fixture"
    np.testing.assert_array_equal(info["idx"].numpy(), fx["idx"])


@pytest.mark.parametrize("path", [p for p in FIXTURES if "deterministic" not in p],
                         ids=[os.path.basename(p)[:-4] for p in FIXTURES if "deterministic" not in p])
def test_oracle_on_reference_paths(path):
    """The oracle evaluated on the reference's own sampled indices (``forced``,
    which the GPU tests use on the GPU's paths) reproduces every value of the
    fixture: the path log-probs (``lp``, including the causal corrections for
    the nodes those paths visit), weights, output and gradients."""
    fx = load(path)
    tol = 2e-2 if str(fx["dtype"]) == "bfloat16" else 1e-5
    out, w, info, (dq, dk, dv) = run_oracle(fx, forced=fx["idx"])
    np.testing.assert_array_equal(info["idx"].numpy(), fx["idx"])
    assert rel(info["lp"].numpy(), fx["lp"]) < tol
    assert rel(out, fx["out"]) < tol
    assert rel(w, fx["weights"]) < tol
    for got, ref in ((dq, fx["dq"]), (dk, fx["dk"]), (dv, fx["dv"])):
        assert rel(got.reshape(ref.shape), ref) < tol
