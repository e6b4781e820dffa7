"""Differentiable float64 restatement of the reference op -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
may import this module, and only as the checker.  The product path
(``treeattention_amd``) never calls it.

Restates ``packages/treeattn-torch/src/treeattn_torch/_tree_mha.py`` on CPU
torch tensors in float64, in the reference's own structure (binary heap tree,
one key per internal node, ``logsigmoid`` decisions), with the Gumbel noise
taken from an explicit uniform tensor ``U`` of shape (B, L, H, S, T, 2)
(``g = -log(-log u)``, the law of the reference's ``-log Exp(1)`` draws at
``_tree_mha.py:109,255``) instead of the global RNG:

* ``sample_non_causal``      -- ``_sample_paths_non_causal``  (``:78-122``)
* ``sample_causal``          -- ``_sample_paths_causal``      (``:125-268``): the
  bottom-up boundary log-masses (fully allowed off-path subtrees weigh their
  leaf count, ``:173-183``), and the top-down corrected decisions that apply
  only while every (batch, head, sample) lane of the query sits on the
  boundary path (``:204-207``)
* ``deterministic_attention`` -- ``_deterministic_attention`` (``:271-321``)
* ``hierarchical_attention`` -- the dispatch (``:324-413``), including the
  causal hybrid (queries ``t < S`` exact, ``:379-385``) and the invalid-index
  mask (``:396-397``).

Autograd through these functions gives the reference's gradients for fixed
sampled directions.  Pinned by the reference's own outputs on the fixtures in
``tests/golden/`` (``tests/test_golden.py``), which ``tests/golden/make_golden.py``
wrote by running the reference with the same uniforms.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

_NEG_INF = float("-inf")


def _gumbel(U) -> torch.Tensor:
    u = torch.as_tensor(np.asarray(U), dtype=torch.float64)
    return -torch.log(-torch.log(u))


def _first_argmax(score: torch.Tensor) -> torch.Tensor:
    """Index of the first maximum along the last axis (torch.argmax's tie rule)."""
    return torch.argmax(score, dim=-1)


def _margin(score: torch.Tensor) -> torch.Tensor:
    s, _ = torch.sort(score, dim=-1, descending=True)
    return (s[..., 0] - s[..., 1]).detach()


def _node_dots(q_lbhd: torch.Tensor, k: torch.Tensor, nodes: torch.Tensor) -> torch.Tensor:
    """``q . k[nodes]`` per (..., b, h, s); ``nodes`` (..., B, H, S), ``q`` broadcast over S."""
    K, B, H, D = k.shape
    kb = k.permute(1, 2, 0, 3)  # (B, H, K, D)
    lead = nodes.shape[:-3]
    kexp = kb.reshape((1,) * len(lead) + (B, H, K, D)).expand(*lead, B, H, K, D)
    idx = nodes.clamp(0, K - 1).unsqueeze(-1).expand(*nodes.shape, D)
    kg = torch.gather(kexp, -2, idx)
    return (q_lbhd.unsqueeze(-2) * kg).sum(-1)


def _forced_dirs(forced, d: int, T: int):
    """Direction at depth ``d`` of the given leaves: bit ``T-1-d`` (``node <- 2 node + 1 + dir``)."""
    return (torch.as_tensor(np.asarray(forced), dtype=torch.long) >> (T - 1 - d)) & 1


def sample_non_causal(q: torch.Tensor, k: torch.Tensor, num_leaves: int, U, forced=None):
    """``_sample_paths_non_causal`` (``_tree_mha.py:78-122``).

    ``q`` (L, B, H, D), ``k`` (K, B, H, D); ``U`` (B, L, H, S, T, 2).
    Returns ``idx`` (L, B, H, S), differentiable ``lp`` and per-decision margins.
    ``forced`` (L, B, H, S) leaf ids: take these paths instead of the
    Gumbel-max decisions (the log-probs and margins are those of the forced
    paths), to evaluate the op on paths another implementation sampled.
    """
    L, B, H, _ = q.shape
    K = num_leaves - 1
    T = (num_leaves - 1).bit_length() if num_leaves > 1 else 0
    S = np.asarray(U).shape[3]
    g = _gumbel(U).permute(1, 0, 2, 3, 4, 5)  # (L, B, H, S, T, 2)
    nodes = torch.zeros(L, B, H, S, dtype=torch.long)
    acc = torch.zeros(L, B, H, S, dtype=q.dtype)
    margins = torch.full((L, B, H, S, max(T, 1)), math.inf, dtype=torch.float64)
    for d in range(T):
        valid = nodes < K
        x = _node_dots(q, k, nodes)
        lp = torch.stack([F.logsigmoid(x), F.logsigmoid(-x)], dim=-1)
        score = lp.detach() + g[..., d, :]
        dirs = _first_argmax(score) if forced is None else _forced_dirs(forced, d, T)
        margins[..., d] = _margin(score)
        chosen = torch.gather(lp, -1, dirs.unsqueeze(-1)).squeeze(-1)
        acc = acc + torch.where(valid, chosen, torch.full_like(chosen, _NEG_INF))
        nodes = 2 * nodes + 1 + dirs
    return nodes - K, acc, margins


def sample_causal(q: torch.Tensor, k: torch.Tensor, num_leaves: int, U, offset: int = 0, forced=None):
    """``_sample_paths_causal`` (``_tree_mha.py:125-268``).

    ``q`` (L', B, H, D) are the queries at absolute positions
    ``offset .. offset + L' - 1``; ``U`` (B, L, H, S, T, 2) is indexed by the
    absolute position.  Returns ``idx`` (L', B, H, S), differentiable ``lp``,
    margins and ``dstar`` (L',): the first depth at which not every lane of
    the query sits on the boundary path (``T`` if none), i.e. where the
    reference stops correcting.  ``forced`` (L', B, H, S) leaf ids: take these
    paths instead of the Gumbel-max decisions; the corrections still follow
    the reference's rule for the nodes the forced paths visit.
    """
    Lq, B, H, _ = q.shape
    K = num_leaves - 1
    T = (num_leaves - 1).bit_length() if num_leaves > 1 else 0
    S = np.asarray(U).shape[3]
    g = _gumbel(U)  # (B, L, H, S, T, 2)
    idx_all, lp_all = [], []
    margins = torch.full((Lq, B, H, S, max(T, 1)), math.inf, dtype=torch.float64)
    dstar = np.full(Lq, T, dtype=np.int64)
    for t in range(Lq):
        c = t + offset
        q_t = q[t]  # (B, H, D)
        # pass 1: boundary path and its bottom-up log-masses (:145-196)
        bnodes = []
        node = 0
        for d in range(T):
            if node >= K:
                break
            bnodes.append(node)
            node = 2 * node + 1 + ((c >> (T - 1 - d)) & 1)
        P = len(bnodes)
        xb = torch.einsum("bhd,pbhd->bhp", q_t, k[torch.tensor(bnodes, dtype=torch.long)])
        mass = torch.zeros(B, H, dtype=q.dtype)
        M = [None] * P
        for d in range(P - 1, -1, -1):
            direction = (c >> (T - 1 - d)) & 1
            n_sub = 1 << (T - 1 - d)
            lpl, lpr = F.logsigmoid(xb[..., d]), F.logsigmoid(-xb[..., d])
            if direction == 0:
                on, off, moff = lpl, lpr, torch.full_like(mass, _NEG_INF)
            else:
                on, off, moff = lpr, lpl, torch.full_like(mass, math.log(n_sub))
            M[d] = torch.logsumexp(torch.stack([mass + on, moff + off]), dim=0)
            mass = M[d]
        # pass 2: top-down, corrected while every lane is on the boundary (:198-262)
        nodes = torch.zeros(B, H, S, dtype=torch.long)
        acc = torch.zeros(B, H, S, dtype=q.dtype)
        for d in range(T):
            on_b = d < P and bool(torch.all(nodes == bnodes[d]))
            if not on_b and dstar[t] == T:
                dstar[t] = d
            x = _node_dots(q_t, k, nodes)  # (B, H, S)
            lpl, lpr = F.logsigmoid(x), F.logsigmoid(-x)
            if on_b:
                direction = (c >> (T - 1 - d)) & 1
                mparent = M[d].unsqueeze(-1)
                mchild = M[d + 1].unsqueeze(-1) if d + 1 < P else torch.zeros(B, H, 1, dtype=q.dtype)
                n_sub = 1 << (T - 1 - d)
                if direction == 0:
                    ml, mr = mchild, torch.full_like(mchild, _NEG_INF)
                else:
                    ml, mr = torch.full_like(mchild, math.log(n_sub)), mchild
                lpl = ml + lpl - mparent
                lpr = mr + lpr - mparent
            lp = torch.stack([lpl, lpr], dim=-1)
            score = lp.detach() + g[:, c, :, :, d, :]
            dirs = _first_argmax(score) if forced is None else _forced_dirs(np.asarray(forced)[t], d, T)
            margins[t, ..., d] = _margin(score)
            acc = acc + torch.gather(lp, -1, dirs.unsqueeze(-1)).squeeze(-1)
            nodes = 2 * nodes + 1 + dirs
        idx_all.append(nodes - K)
        lp_all.append(acc)
    return torch.stack(idx_all), torch.stack(lp_all), margins, dstar


def leaf_logprobs(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """``log P(leaf n)`` for every leaf of the binary heap tree, (L, B, H, N), as built
    level by level in ``_deterministic_attention`` (``_tree_mha.py:286-306``)."""
    L, B, H, _ = q.shape
    K = k.shape[0]
    T = K.bit_length() if K else 0
    lpp = torch.zeros(L, B, H, 1, dtype=q.dtype)
    for d in range(T):
        kd = k[(1 << d) - 1:(1 << (d + 1)) - 1]  # (2^d, B, H, D)
        x = torch.einsum("lbhd,nbhd->lbhn", q, kd)
        ch = torch.stack([F.logsigmoid(x), F.logsigmoid(-x)], dim=-1)
        lpp = (lpp.unsqueeze(-1) + ch).reshape(L, B, H, -1)
    return lpp


def deterministic_attention(q, k, v, is_causal: bool):
    """``_deterministic_attention`` (``_tree_mha.py:271-321``) for ``N = 2^T`` leaves.

    Returns ``out`` (L, B, H, D) and the leaf weights (L, B, H, N): ``exp`` of the
    path log-probabilities, or (causal) their softmax over leaves ``n <= l``.
    """
    L = q.shape[0]
    N = v.shape[0]
    lpp = leaf_logprobs(q, k)[..., :N]
    if is_causal:
        mask = torch.arange(N).view(1, N) > torch.arange(L).view(L, 1)
        lpp = lpp.masked_fill(mask[:, None, None, :], _NEG_INF)
        w = torch.softmax(lpp, dim=-1)
    else:
        w = torch.exp(lpp)
    return torch.einsum("lbhn,nbhd->lbhd", w, v), w


def hierarchical_attention(query, key, value, num_heads: int, is_causal: bool = False,
                           mode: str = "stochastic", num_samples: int = 64, U=None, forced=None):
    """``hierarchical_attention`` (``_tree_mha.py:324-413``) on float64 tensors.

    ``query`` (L, B, E), ``key`` (N-1, B, E), ``value`` (N, B, E); ``U`` the
    uniforms (B, L, H, S, T, 2) for stochastic mode.  Returns ``(out (L, B, E),
    weights)`` with the reference's shapes (hybrid causal: weights of the
    stochastic rows only) and, for stochastic mode, a dict with ``idx``,
    ``margins`` and ``dstar`` of the sampled rows.  ``forced``: leaf ids of
    the sampled rows (``(L - S, B, H, S)`` for the causal hybrid, else
    ``(L, B, H, S)``) to evaluate on instead of sampling.
    """
    L, B, E = query.shape
    N = value.shape[0]
    H = num_heads
    D = E // H
    K = N - 1
    q = query.reshape(L, B, H, D)
    k = key.reshape(K, B, H, D)
    v = value.reshape(N, B, H, D)
    if mode == "deterministic":
        out, w = deterministic_attention(q, k, v, is_causal)
        return out.reshape(L, B, E), w, {}
    S = num_samples
    info = {}
    hybrid = is_causal and L > S
    if hybrid:
        out_det, _ = deterministic_attention(q[:S], k, v, True)
        idx, lp, margins, dstar = sample_causal(q[S:], k, N, U, offset=S, forced=forced)
        info["dstar"] = dstar
    elif is_causal:
        idx, lp, margins, dstar = sample_causal(q, k, N, U, offset=0, forced=forced)
        info["dstar"] = dstar
    else:
        idx, lp, margins = sample_non_causal(q, k, N, U, forced=forced)
    info.update(idx=idx, margins=margins, lp=lp.detach())
    valid = (idx >= 0) & (idx < N)
    lp = lp.masked_fill(~valid, _NEG_INF)
    w = torch.softmax(lp, dim=-1)
    vb = v.permute(1, 2, 0, 3)  # (B, H, N, D)
    lead = idx.shape[0]
    vexp = vb.unsqueeze(0).expand(lead, B, H, N, D)
    gi = idx.clamp(0, N - 1).unsqueeze(-1).expand(*idx.shape, D)
    gathered = torch.gather(vexp, -2, gi)
    out_sto = torch.einsum("lbhs,lbhsd->lbhd", w, gathered)
    out = torch.cat([out_det, out_sto], dim=0) if hybrid else out_sto
    return out.reshape(L, B, E), w, info
