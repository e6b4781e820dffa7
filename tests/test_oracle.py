"""Pins the CPU oracle (``oracle/tree_oracle.py``) before anything is checked against it.

Each check is chosen so a plausible slip (a dropped term, a wrong sign or
index, a transposed operand) fails: known-answer vectors, closed forms,
brute-force enumeration, sampling frequencies, and torch autograd through an
independent restatement.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import tree_oracle as O


# ---------------------------------------------------------------- Philox ----

# Random123 known-answer vectors for philox4x32-10 (kat_vectors, Salmon et al.).
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", PHILOX_KAT)
def test_philox_known_answers(ctr, key, expect):
    out = O.philox4x32_10(np.array([ctr], dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert tuple(int(x) for x in out[0]) == expect


def test_uniforms_open_interval_and_layout():
    u = O.uniforms(0, (3, 5, 7))
    assert u.dtype == np.float32 and u.shape == (3, 5, 7)
    assert (u > 0).all() and (u < 1).all()
    flat = O.uniforms(0, (105,))
    np.testing.assert_array_equal(u.reshape(-1), flat)  # row-major flat index
    assert not np.array_equal(O.uniforms(1, (105,)), flat)
    # mean/variance of U(0,1) within 5 sigma
    big = O.uniforms(7, (200000,)).astype(np.float64)
    assert abs(big.mean() - 0.5) < 5 * math.sqrt(1 / 12 / big.size)
    assert abs(big.var() - 1 / 12) < 0.002
    # the extreme words map strictly inside (0, 1) in float32 (so -log(-log u) is finite)
    ext = O.word_uniform(np.array([0, 1, 0x1FF, 0x200, 0xFFFFFDFF, 0xFFFFFE00, 0xFFFFFFFF], dtype=np.uint32))
    assert ext[0] == np.float32(2.0**-24) and ext[-1] == np.float32(1 - 2.0**-24) and ext[-1] < 1
    assert ext[2] == ext[0] and ext[3] == np.float32(1.5 * 2.0**-23) and ext[-2] == ext[-1] and ext[-3] < ext[-2]
    assert np.isfinite(O.gumbel(ext)).all()


# ------------------------------------------------------------------ Haar ----


def test_haar_closed_form_inorder():
    rng = np.random.default_rng(0)
    n = 16
    m = rng.standard_normal((n, 3))
    coef = O.haar_inorder(m)
    for j in range(n - 1):
        p = j + 1
        ell = (p & -p).bit_length() - 1
        w = 1 << ell
        expect = (m[p - w:p].mean(axis=0) - m[p:p + w].mean(axis=0)) / 2
        np.testing.assert_allclose(coef[j], expect, rtol=1e-12, atol=1e-12)
    # the reference root decision uses the finest leaf-pair difference
    np.testing.assert_allclose(coef[0], (m[0] - m[1]) / 2)


def test_haar_adjoint_identity():
    rng = np.random.default_rng(1)
    for n in (2, 4, 32):
        x = rng.standard_normal((n, 2))
        y = rng.standard_normal((n - 1, 2))
        lhs = np.sum(O.haar_inorder(x) * y)
        rhs = np.sum(x * O.haar_inorder_adjoint(y))
        assert abs(lhs - rhs) < 1e-12


def test_haar_invertible_with_global_mean():
    rng = np.random.default_rng(2)
    n = 8
    m = rng.standard_normal(n)
    rows = [O.haar_inorder(np.eye(n)[i]) for i in range(n)]
    A = np.concatenate([np.full((n, 1), 1.0 / n), np.stack(rows)], axis=1)  # x -> (mean, coef)
    assert np.linalg.matrix_rank(A) == n
    np.testing.assert_allclose(m @ A[:, 1:], O.haar_inorder(m))


def test_natural_binary_summaries_are_subtree_haar():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((1, 16, 1, 4))
    C = O.pool_natural(k, 2, 2)  # NL = 8, T = 3
    off = O.level_offsets(2, 3)
    m = k[0, :, 0].reshape(8, 2, 4).mean(axis=1)
    # depth-1 node 1 (level-2 children rows 2,3) covers blocks 4..7
    left, right = C[0, 0, off[2] + 2], C[0, 0, off[2] + 3]
    np.testing.assert_allclose(left - right, (m[4:6].mean(0) - m[6:8].mean(0)) / 2)
    np.testing.assert_allclose(C[0, 0, off[1]], m[:4].mean(0) / 2)


def test_pool_adjoints_by_inner_product():
    rng = np.random.default_rng(4)
    for b, LB, mode in ((2, 1, "compat"), (2, 4, "compat"), (4, 2, "natural"), (2, 2, "natural")):
        L = 32
        k = rng.standard_normal((2, L, 2, 3))
        C = O.summaries(k, b, LB, mode)
        dC = rng.standard_normal(C.shape)
        lhs = np.sum(C * dC)
        rhs = np.sum(k * O.pool_adjoint(dC, L, b, LB, mode))
        assert abs(lhs - rhs) < 1e-10, (b, LB, mode)


# ---------------------------------------------- brute-force path sampling ----


def _leaf_logprobs_binary(q, knodes):
    """Exact log P(leaf) for every leaf of a heap-indexed binary tree."""
    K = knodes.shape[0]
    N = K + 1
    T = N.bit_length() - 1
    out = np.zeros(N)
    for leaf in range(N):
        node, lp = 0, 0.0
        for d in range(T):
            bit = (leaf >> (T - 1 - d)) & 1
            x = float(q @ knodes[node])
            lp += -np.logaddexp(0, -x) if bit == 0 else -np.logaddexp(0, x)
            node = 2 * node + 1 + bit
        out[leaf] = lp
    return out


def test_ref_sampler_logprobs_match_enumeration():
    rng = np.random.default_rng(5)
    L, B, H, D, N, S = 6, 1, 2, 4, 8, 5
    q = rng.standard_normal((L, B, H, D))
    kn = rng.standard_normal((N - 1, B, H, D))
    U = O.uniforms(11, (L, B, H, S, 3, 2))
    idx, lp = O.ref_sample_paths_non_causal(q, kn, O.gumbel(U))
    for l in range(L):
        for h in range(H):
            exact = _leaf_logprobs_binary(q[l, 0, h], kn[:, 0, h])
            np.testing.assert_allclose(lp[l, 0, h], exact[idx[l, 0, h]], rtol=1e-12)
            assert abs(np.logaddexp.reduce(exact)) < 1e-12  # probabilities sum to one


def test_ref_sampler_gumbel_frequencies_chi_square():
    rng = np.random.default_rng(6)
    D, N, S = 3, 8, 40000
    q = rng.standard_normal((1, 1, 1, D))
    kn = rng.standard_normal((N - 1, 1, 1, D))
    U = O.uniforms(3, (1, 1, 1, S, 3, 2))
    idx, _ = O.ref_sample_paths_non_causal(q, kn, O.gumbel(U))
    p = np.exp(_leaf_logprobs_binary(q[0, 0, 0], kn[:, 0, 0]))
    counts = np.bincount(idx.reshape(-1), minlength=N)
    chi2 = np.sum((counts - S * p) ** 2 / (S * p))
    assert chi2 < 30.0  # 7 dof: P(chi2 > 30) ~ 1e-4


def test_generalized_reduces_to_reference_binary_lb1():
    rng = np.random.default_rng(7)
    B, L, H, D, S = 2, 16, 3, 8, 6
    q = rng.standard_normal((B, L, H, D))
    k = rng.standard_normal((B, L, H, D))
    v = rng.standard_normal((B, L, H, D))
    U = O.uniforms(0, (B, L, H, S, 4, 2))
    # adapter path of the reference: Haar(k) in-order, read in heap order
    knodes_sbhd = O.haar_inorder(k.transpose(1, 0, 2, 3))  # (L-1,B,H,D)
    ref_out, ref_w, ref_idx = O.ref_forward_non_causal(
        q.transpose(1, 0, 2, 3), knodes_sbhd, v.transpose(1, 0, 2, 3),
        O.gumbel(U).transpose(1, 0, 2, 3, 4, 5))
    C = O.pool_compat(k, 1)
    out, w, idx, lp, margins = O.tree_forward(q, k, v, C, 2, 1, U, causal=False)
    np.testing.assert_array_equal(idx, ref_idx.transpose(1, 0, 2, 3))
    np.testing.assert_allclose(w, ref_w.transpose(1, 0, 2, 3), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(out, ref_out.transpose(1, 0, 2, 3), rtol=1e-10, atol=1e-12)


def _leaf_logprobs_bary(qv, C, b, T):
    off = O.level_offsets(b, T)
    nl = b**T
    out = np.zeros(nl)
    for leaf in range(nl):
        lp = 0.0
        for d in range(T):
            node = leaf // b ** (T - d)
            j = (leaf // b ** (T - 1 - d)) % b
            x = np.array([qv @ C[off[d + 1] + b * node + jj] for jj in range(b)])
            lp += x[j] - np.logaddexp.reduce(x)
        out[leaf] = lp
    return out


def test_branching4_logprobs_and_frequencies():
    rng = np.random.default_rng(8)
    b, LB, D, S = 4, 2, 4, 30000
    L = LB * 16  # NL=16, T=2
    q = rng.standard_normal((1, L, 1, D))
    k = 2 * rng.standard_normal((1, L, 1, D))
    C = O.pool_natural(k, b, LB)
    U = O.uniforms(5, (1, L, 1, S, 2, b))
    idx, lp, _ = O.tree_sample(q, C, b, LB, U, causal=False)
    exact = _leaf_logprobs_bary(q[0, 0, 0], C[0, 0], b, 2)
    np.testing.assert_allclose(lp[0, 0, 0], exact[idx[0, 0, 0]], rtol=1e-12, atol=1e-12)
    counts = np.bincount(idx[0, 0, 0], minlength=16)
    p = np.exp(exact)
    chi2 = np.sum((counts - S * p) ** 2 / (S * p))
    assert chi2 < 45.0  # 15 dof


def test_causal_restricted_distribution():
    rng = np.random.default_rng(9)
    b, LB, D, S = 2, 2, 4, 30000
    L = LB * 8  # NL=8, T=3
    q = rng.standard_normal((1, L, 1, D))
    k = 2 * rng.standard_normal((1, L, 1, D))
    C = O.pool_natural(k, b, LB)
    U = O.uniforms(6, (1, L, 1, S, 3, b))
    idx, lp, _ = O.tree_sample(q, C, b, LB, U, causal=True)
    for t in (0, 5, 9, 15):
        blk = t // LB
        assert idx[0, t, 0].max() <= blk
        exact = _leaf_logprobs_bary(q[0, t, 0], C[0, 0], b, 3)
        allowed = exact[: blk + 1]
        logA = np.logaddexp.reduce(allowed)
        # accumulated corrected log-probs = log P(leaf) - log A_root
        np.testing.assert_allclose(lp[0, t, 0], exact[idx[0, t, 0]] - logA, rtol=1e-9, atol=1e-9)
        if blk >= 1:
            p = np.exp(allowed - logA)
            counts = np.bincount(idx[0, t, 0], minlength=blk + 1)
            chi2 = np.sum((counts - S * p) ** 2 / (S * p))
            assert chi2 < 20.0 + 3 * blk


def test_leaf_attention_matches_textbook_masked_softmax():
    rng = np.random.default_rng(10)
    B, L, H, D, S, LB = 1, 16, 2, 8, 3, 4
    q, k, v = (rng.standard_normal((B, L, H, D)) for _ in range(3))
    idx = rng.integers(0, 4, size=(B, L, H, S))
    for causal in (False, True):
        if causal:
            idx = np.minimum(idx, np.arange(L)[None, :, None, None] // LB)
        o_s, _ = O.leaf_attention(q, k, v, idx, LB, causal, 0.3)
        for l in (0, 5, 15):
            for h in range(H):
                for s in range(S):
                    blk = idx[0, l, h, s]
                    toks = np.arange(blk * LB, blk * LB + LB)
                    if causal:
                        toks = toks[toks <= l]
                    qt = torch.tensor(q[0, l, h][None, None, None])
                    kt = torch.tensor(k[0, toks, h][None, None])
                    vt = torch.tensor(v[0, toks, h][None, None])
                    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=0.3)
                    np.testing.assert_allclose(o_s[0, l, h, s], ref[0, 0, 0].numpy(), rtol=1e-10)


# ------------------------------------------------------------- backward ----


def _torch_forward_fixed_paths(q, k, v, idx, b, LB, causal, tree_mode, scale):
    """Independent torch restatement with the sampled paths held fixed."""
    B, L, H, D = q.shape
    nl = L // LB
    T = O.tree_depth(nl, b)
    m = k.reshape(B, nl, LB, H, D).mean(dim=2).permute(0, 2, 1, 3)  # (B,H,NL,D)
    # child logits along each path, computed straight from subtree means
    if tree_mode == "natural":
        def child_summary(level, node_ids):  # node ids at `level` (1..T)
            per = nl // b**level
            sub = m.reshape(B, H, b**level, per, D).mean(dim=3) / 2
            return sub
        levels = [child_summary(lam, None) for lam in range(1, T + 1)]
    else:  # compat: Haar over block means in the reference's loop, heap read
        out = m.permute(2, 0, 1, 3)
        n = nl
        for level in range(n.bit_length() - 1):
            step = 1 << level
            base = torch.arange(n >> (level + 1)) * (2 * step)
            a_, b_ = out[base], out[base + step]
            out = out.clone()
            out[base] = (a_ + b_) / 2
            out[base + step] = (a_ - b_) / 2
        kn = out[1:].permute(1, 2, 0, 3)  # (B,H,K,D)
        levels = []
        for lam in range(1, T + 1):
            d = lam - 1
            nodes = kn[:, :, (1 << d) - 1:(1 << (d + 1)) - 1]
            levels.append(torch.stack([nodes / 2, -nodes / 2], dim=3).reshape(B, H, 2 << d, D))
    S = idx.shape[-1]
    lp = torch.zeros(B, L, H, S, dtype=q.dtype)
    leaf = torch.as_tensor(idx)
    for d in range(T):
        node = leaf // b ** (T - d)
        jst = (leaf // b ** (T - 1 - d)) % b
        lvl = levels[d]  # (B,H,b**(d+1),D)
        x = torch.einsum("blhd,bhnd->blhn", q, lvl)  # (B,L,H,b**(d+1))
        cols = b * node.unsqueeze(-1) + torch.arange(b)
        xs = torch.gather(x.unsqueeze(3).expand(B, L, H, S, x.shape[-1]), -1, cols)
        logp = xs - torch.logsumexp(xs, dim=-1, keepdim=True)
        lp = lp + torch.gather(logp, -1, jst.unsqueeze(-1)).squeeze(-1)
        if causal:  # per-query constant: must not change any gradient
            lp = lp + 0.37 * x.sum(dim=-1, keepdim=True).tanh()
    w = torch.softmax(lp, dim=-1)
    tok = leaf.unsqueeze(-1) * LB + torch.arange(LB)
    bi = torch.arange(B)[:, None, None, None, None]
    hi = torch.arange(H)[None, None, :, None, None]
    Kg, Vg = k[bi, tok, hi], v[bi, tok, hi]
    z = scale * torch.einsum("blhd,blhsjd->blhsj", q, Kg)
    if causal:
        z = z.masked_fill(tok > torch.arange(L)[None, :, None, None, None], float("-inf"))
    a = torch.softmax(z, dim=-1)
    o_s = torch.einsum("blhsj,blhsjd->blhsd", a, Vg)
    return torch.einsum("blhs,blhsd->blhd", w, o_s)


@pytest.mark.parametrize("b,LB,causal,mode", [
    (2, 1, False, "compat"), (2, 4, True, "compat"), (4, 2, False, "natural"),
    (4, 4, True, "natural"), (2, 2, True, "natural"),
])
def test_backward_matches_autograd(b, LB, causal, mode):
    rng = np.random.default_rng(12)
    B, H, D, S = 2, 2, 8, 5
    L = LB * b**2 * (2 if b == 2 else 1)
    q, k, v, g = (rng.standard_normal((B, L, H, D)) for _ in range(4))
    nl = L // LB
    T = O.tree_depth(nl, b)
    U = O.uniforms(4, (B, L, H, S, T, b))
    res = O.attention_fwd_bwd(q, k, v, g, b, LB, U, causal, mode, scale=0.4)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    out = _torch_forward_fixed_paths(qt, kt, vt, res["idx"], b, LB, causal, mode, 0.4)
    np.testing.assert_allclose(out.detach().numpy(), res["out"], rtol=1e-10, atol=1e-12)
    out.backward(torch.tensor(g))
    np.testing.assert_allclose(qt.grad.numpy(), res["dq"], rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(kt.grad.numpy(), res["dk"], rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(vt.grad.numpy(), res["dv"], rtol=1e-9, atol=1e-10)


def test_backward_finite_differences_reference_mode():
    rng = np.random.default_rng(13)
    B, L, H, D, S = 1, 8, 1, 4, 3
    q, k, v, g = (rng.standard_normal((B, L, H, D)) for _ in range(4))
    U = O.uniforms(2, (B, L, H, S, 3, 2))
    base = O.attention_fwd_bwd(q, k, v, g, 2, 1, U, False, "compat")
    eps = 1e-6
    for name, x in (("dq", q), ("dk", k), ("dv", v)):
        for _ in range(4):
            i = tuple(int(rng.integers(0, n)) for n in x.shape)
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            args = {"dq": (q, k, v), "dk": (q, k, v), "dv": (q, k, v)}[name]
            def loss(xx):
                qq, kk, vv = [xx if a is x else a for a in args]
                r = O.attention_fwd_bwd(qq, kk, vv, None, 2, 1, U, False, "compat")
                assert np.array_equal(r["idx"], base["idx"])  # paths unchanged
                return np.sum(r["out"] * g)
            fd = (loss(xp) - loss(xm)) / (2 * eps)
            assert abs(fd - base[name][i]) < 1e-6 * max(1, abs(fd)), (name, i, fd, base[name][i])


# ------------------------------------------------------- path log-probs ----


@pytest.mark.parametrize("b", [2, 4, 8])
@pytest.mark.parametrize("LB", [1, 3])
def test_path_logprobs_pinned(b, LB):
    """``path_logprobs`` (``_tree_mha.py:112-117``: the chosen child's log-prob
    summed along the path) three ways: against brute-force enumeration of every
    leaf block's path, against the sampler's own accumulated log-probs
    (non-causal), and against the exact causal sampler's corrected log-probs
    plus ``log A_root`` (the allowed mass), with N != L."""
    rng = np.random.default_rng(100 + 10 * b + LB)
    T = 2 if b == 8 else 3
    nl = b**T
    N = LB * nl
    B, H, D, S = 2, 2, 4, 6
    mode = "compat" if b == 2 and LB == 3 else "natural"
    k = 1.5 * rng.standard_normal((B, N, H, D))
    C = O.summaries(k, b, LB, mode)
    # (1) brute force on random leaf blocks
    L = 5
    q = rng.standard_normal((B, L, H, D))
    idx = rng.integers(0, nl, size=(B, L, H, S))
    lp = O.path_logprobs(q, C, b, nl, idx)
    for bb in range(B):
        for h in range(H):
            for l in range(L):
                exact = _leaf_logprobs_bary(q[bb, l, h], C[bb, h], b, T)
                assert abs(np.logaddexp.reduce(exact)) < 1e-12
                np.testing.assert_allclose(lp[bb, l, h], exact[idx[bb, l, h]], rtol=1e-12, atol=1e-12)
    # (2) the non-causal sampler's accumulated log-probs
    U = O.uniforms(7, (B, L, H, S, T, b))
    idx_s, lp_s, _ = O.tree_sample(q, C, b, LB, U, causal=False, N=N)
    np.testing.assert_allclose(O.path_logprobs(q, C, b, nl, idx_s), lp_s, rtol=1e-12, atol=1e-12)
    # (3) exact causal mode, L < N (bottom-right aligned): lp_sampler + log A_root = path log-prob
    Lc = N - 2 * LB - 1
    qc = rng.standard_normal((B, Lc, H, D))
    Uc = O.uniforms(8, (B, Lc, H, S, T, b))
    idx_c, lp_c, _ = O.tree_sample(qc, C, b, LB, Uc, causal=True, N=N)
    full = O.path_logprobs(qc, C, b, nl, idx_c)
    for bb in range(B):
        for h in range(H):
            for l in (0, Lc // 2, Lc - 1):
                blk = (l + N - Lc) // LB
                assert idx_c[bb, l, h].max() <= blk
                exact = _leaf_logprobs_bary(qc[bb, l, h], C[bb, h], b, T)
                logA = np.logaddexp.reduce(exact[:blk + 1])
                np.testing.assert_allclose(lp_c[bb, l, h] + logA, full[bb, l, h], rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("b,LB,causal,mode,NmL", [
    (2, 1, False, "compat", 0), (2, 4, True, "compat", 8), (4, 2, False, "natural", 0),
    (4, 4, True, "natural", 0), (2, 3, True, "natural", 5),
])
def test_head_fwd_bwd_matches_explicit(b, LB, causal, mode, NmL):
    """The per-head, block-organized ``head_fwd_bwd`` against ``leaf_attention``,
    ``path_logprobs`` / ``sample_weights`` and ``tree_backward`` (each pinned
    above) on the same paths, every output and gradient."""
    rng = np.random.default_rng(21)
    H, D, S = 2, 8, 5
    nl = b**3
    N = LB * nl
    L = N - NmL
    q, g = (rng.standard_normal((1, L, H, D)) for _ in range(2))
    k, v = (rng.standard_normal((1, N, H, D)) for _ in range(2))
    U = O.uniforms(4, (1, L, H, S, 3, b))
    C = O.summaries(k, b, LB, mode)
    idx, _, _ = O.tree_sample(q, C, b, LB, U, causal, N=N)
    w = O.sample_weights(O.path_logprobs(q, C, b, nl, idx))
    o_s, _ = O.leaf_attention(q, k, v, idx, LB, causal, 0.3)
    out = np.einsum("blhs,blhsd->blhd", w, o_s)
    dq, dC, dkl, dv = O.tree_backward(q, k, v, C, b, LB, idx, w, g, causal, 0.3)
    for h in range(H):
        r = O.head_fwd_bwd(q[0, :, h], k[0, :, h], v[0, :, h], g[0, :, h], C[0, h], b, LB, idx[0, :, h], causal, 0.3)
        np.testing.assert_allclose(r["weights"], w[0, :, h], rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(r["out"], out[0, :, h], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["dq"], dq[0, :, h], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["dC"], dC[0, h], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["dk_leaf"], dkl[0, :, h], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["dv"], dv[0, :, h], rtol=1e-10, atol=1e-12)


def test_uniforms_at_matches_full_tensor():
    u = O.uniforms(9, (3, 7, 5))
    flat = np.array([0, 1, 2, 3, 4, 17, 50, 101, 104])
    np.testing.assert_array_equal(O.uniforms_at(9, flat), u.reshape(-1)[flat])


def test_path_logits_gathered_equals_dense():
    """``path_logits``' gathered form (large trees) against the dense product."""
    rng = np.random.default_rng(31)
    Q = rng.standard_normal((300, 16))
    C = rng.standard_normal((200000, 16))
    cols = rng.integers(0, C.shape[0], size=(300, 5, 2))
    got = O.path_logits(Q, C, cols)  # 300 * 200000 > 2^25: the gathered form
    ref = np.einsum("ld,lsjd->lsj", Q, C[cols])
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    small = O.path_logits(Q, C[:1000], cols % 1000)  # the dense form
    np.testing.assert_allclose(small, np.einsum("ld,lsjd->lsj", Q, C[cols % 1000]), rtol=1e-12, atol=1e-12)
