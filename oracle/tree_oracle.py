"""CPU oracle for stochastic tree attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed CPU
baseline).  The product path (``treeattention_amd``) never calls it; it fails
loudly when the HIP library is missing.

Everything is float64 numpy on explicit inputs:

* ``philox4x32_10`` / ``uniforms``: the counter RNG that fills the caller
  uniform tensor (Salmon et al., "Parallel random numbers: as easy as 1, 2, 3",
  SC'11).  The reference draws its Gumbel noise from torch's global RNG
  (``packages/treeattn-torch/src/treeattn_torch/_tree_mha.py:109``); the build
  replaces that stream with explicit uniforms ``u`` and ``g = -log(-log u)``,
  which is the same Gumbel law (``Exp(1) = -log U``).
* ``haar_inorder``: restates ``haar_internal_node_keys``
  (``packages/attn-bench/src/attn_bench/baselines/_treeattn_common.py:54-86``).
* ``ref_*``: restatements of the reference's own stochastic path in its own
  structure (binary heap tree, one key per node, ``logsigmoid``): sampler
  ``_tree_mha.py:78-122``, combine ``_tree_mha.py:396-407``.
* ``pool_*``, ``tree_forward``, ``tree_backward``: the generalized semantics
  (branching ``b``, leaf block ``LB``) that the HIP kernels implement.  At
  ``b=2, LB=1`` with the ``compat`` summaries they reduce to ``ref_*`` (pinned
  in ``tests/test_oracle.py``).

Parity status per function (what pins it, all in ``tests/test_oracle.py``):

* ``philox4x32_10``: Random123 known-answer vectors.
* ``haar_inorder``: closed form of the in-order layout, orthogonality/inverse,
  ``haar_inorder_adjoint`` by the inner-product identity.
* ``ref_sample_paths_non_causal`` / ``ref_forward_non_causal``: brute-force path
  enumeration (sampled log-probs equal exact path log-probabilities), Gumbel-max
  frequencies against exact leaf probabilities (chi-square), textbook cases.
* ``tree_forward``: reduction to ``ref_forward_non_causal`` at ``b=2, LB=1``;
  brute force for ``b=4`` and causal restriction; leaf block against a
  textbook masked softmax attention.
* ``tree_backward``: torch autograd through an independent torch restatement
  and central finite differences.
* ``pack_paths`` / ``unpack_paths``: the heap walk of the reference
  (``heap_walk``, ``_autograd.py:219,312-315``) on random directions, packed
  depth by depth as the reference does (``_autograd.py:214-216``), and round
  trips; the golden fixtures' sampled indices replayed on the GPU reproduce
  the reference's outputs (``tests/test_gpu_paths.py``).
* Causal mode of the reference (``_tree_mha.py:125-268,379-394``) is NOT
  restated here: the generalized causal semantics below sample exactly from
  the tree distribution restricted to allowed leaves, which the reference's
  coupled sampler does not (see ``causal_boundary_logmass``).
"""

from __future__ import annotations

import math

import numpy as np

# --------------------------------------------------------------------------
# Counter RNG: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11).
# --------------------------------------------------------------------------

PHILOX_M0 = np.uint64(0xD2511F53)
PHILOX_M1 = np.uint64(0xCD9E8D57)
PHILOX_W0 = np.uint32(0x9E3779B9)
PHILOX_W1 = np.uint32(0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """Philox4x32 with 10 rounds.  ``ctr``: (N, 4) uint32, ``key``: (2,) uint32."""
    c = [ctr[:, i].astype(np.uint64) for i in range(4)]
    k0 = np.uint32(key[0])
    k1 = np.uint32(key[1])
    for r in range(10):
        if r > 0:
            k0 = np.uint32((int(k0) + int(PHILOX_W0)) & 0xFFFFFFFF)
            k1 = np.uint32((int(k1) + int(PHILOX_W1)) & 0xFFFFFFFF)
        p0 = PHILOX_M0 * c[0]
        p1 = PHILOX_M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK32
        c = [
            (hi1 ^ c[1] ^ np.uint64(k0)) & _MASK32,
            lo1,
            (hi0 ^ c[3] ^ np.uint64(k1)) & _MASK32,
            lo0,
        ]
    return np.stack(c, axis=1).astype(np.uint32)


def uniforms(seed: int, shape: tuple[int, ...]) -> np.ndarray:
    """Uniforms in (0, 1), float32, identical to the GPU generator.

    Element with flat (row-major) index ``i`` takes word ``i % 4`` of
    ``philox4x32_10(ctr=(lo(i//4), hi(i//4), 0, 0), key=(lo(seed), hi(seed)))``
    and maps it with ``word_uniform``.
    """
    n = int(np.prod(shape)) if len(shape) else 1
    nblk = (n + 3) // 4
    idx = np.arange(nblk, dtype=np.uint64)
    ctr = np.zeros((nblk, 4), dtype=np.uint32)
    ctr[:, 0] = (idx & _MASK32).astype(np.uint32)
    ctr[:, 1] = (idx >> np.uint64(32)).astype(np.uint32)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    words = philox4x32_10(ctr, key).reshape(-1)[:n]
    return word_uniform(words).reshape(shape)


def uniforms_at(seed: int, flat: np.ndarray) -> np.ndarray:
    """The elements of ``uniforms(seed, shape)`` at the given flat (row-major)
    indices, without generating the rest."""
    flat = np.asarray(flat).astype(np.uint64).reshape(-1)
    blk = flat >> np.uint64(2)
    ctr = np.zeros((flat.size, 4), dtype=np.uint32)
    ctr[:, 0] = (blk & _MASK32).astype(np.uint32)
    ctr[:, 1] = (blk >> np.uint64(32)).astype(np.uint32)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    words = philox4x32_10(ctr, key)[np.arange(flat.size), (flat & np.uint64(3)).astype(np.int64)]
    return word_uniform(words)


def word_uniform(words: np.ndarray) -> np.ndarray:
    """32-bit words -> float32 uniforms ``((x >> 9) + 0.5) * 2**-23``: every value
    is exact in float32 and lies in ``[2**-24, 1 - 2**-24]``, strictly inside (0, 1)."""
    u = ((np.asarray(words, dtype=np.uint32) >> np.uint32(9)).astype(np.float64) + 0.5) * (2.0 ** -23)
    return u.astype(np.float32)


def gumbel(u: np.ndarray) -> np.ndarray:
    """``g = -log(-log u)`` in float64 (``_tree_mha.py:109`` draws ``-log Exp(1)``)."""
    u = np.asarray(u, dtype=np.float64)
    return -np.log(-np.log(u))


# --------------------------------------------------------------------------
# Tree geometry
# --------------------------------------------------------------------------


def tree_depth(num_leaf_blocks: int, branching: int) -> int:
    """``T`` with ``branching**T == num_leaf_blocks``; raises otherwise."""
    if num_leaf_blocks < 1 or branching < 2:
        raise ValueError("need num_leaf_blocks >= 1 and branching >= 2")
    t, n = 0, 1
    while n < num_leaf_blocks:
        n *= branching
        t += 1
    if n != num_leaf_blocks:
        raise ValueError(
            f"num_leaf_blocks={num_leaf_blocks} is not a power of branching={branching}"
        )
    return t


def level_offsets(branching: int, depth: int) -> list[int]:
    """Row offset of each level's node summaries, level 1..T, plus the total.

    Summaries are stored level-major: level ``lam`` (``1 <= lam <= T``) holds
    ``branching**lam`` rows starting at ``off[lam]``; ``off[T+1]`` is ``NS``.
    ``off[0]`` is unused (the root has no summary).
    """
    off = [0, 0]
    for lam in range(1, depth + 1):
        off.append(off[-1] + branching**lam)
    return off


# --------------------------------------------------------------------------
# Key summaries ("pooling")
# --------------------------------------------------------------------------


def haar_inorder(m: np.ndarray) -> np.ndarray:
    """In-order Haar coefficients along axis 0, global mean dropped.

    Restates ``haar_internal_node_keys`` (``_treeattn_common.py:65-86``):
    per level, pairs ``(i, i + step)`` become ``((a+b)/2, (a-b)/2)`` in place,
    then index 0 (the global mean) is dropped.
    """
    n = m.shape[0]
    if n < 1 or n & (n - 1):
        raise ValueError(f"haar needs a power-of-two length, got {n}")
    out = np.array(m, dtype=np.float64, copy=True)
    levels = n.bit_length() - 1
    for level in range(levels):
        step = 1 << level
        base = np.arange(n >> (level + 1)) * (2 * step)
        a = out[base].copy()
        b = out[base + step].copy()
        out[base] = (a + b) / 2
        out[base + step] = (a - b) / 2
    return out[1:]


def haar_inorder_adjoint(dcoef: np.ndarray) -> np.ndarray:
    """Transpose of ``haar_inorder`` (the per-level 2x2 map is symmetric)."""
    n = dcoef.shape[0] + 1
    dout = np.zeros((n,) + dcoef.shape[1:], dtype=np.float64)
    dout[1:] = dcoef
    levels = n.bit_length() - 1
    for level in reversed(range(levels)):
        step = 1 << level
        base = np.arange(n >> (level + 1)) * (2 * step)
        da = dout[base].copy()
        dd = dout[base + step].copy()
        dout[base] = (da + dd) / 2
        dout[base + step] = (da - dd) / 2
    return dout


def block_means(k: np.ndarray, leaf_block: int) -> np.ndarray:
    """``(B, L, H, D) -> (B, H, NL, D)`` mean keys of each leaf block."""
    B, L, H, D = k.shape
    nl = L // leaf_block
    return k.astype(np.float64).reshape(B, nl, leaf_block, H, D).mean(axis=2).transpose(0, 2, 1, 3)


def nodekeys_to_summaries(knodes: np.ndarray) -> np.ndarray:
    """Heap-indexed node keys ``(B, H, K, D)`` -> child summaries ``(B, H, NS, D)``.

    Binary node ``n`` (heap order: root 0, children ``2n+1+dir``,
    ``_tree_mha.py:119``) with key ``k_n`` gets child summaries
    ``+k_n/2`` (left) and ``-k_n/2`` (right), so that
    ``softmax(q.k/2, -q.k/2) = (sigmoid(q.k), sigmoid(-q.k))``, the
    reference's ``[logsigmoid(s), logsigmoid(-s)]`` (``_tree_mha.py:107``).
    """
    B, H, K, D = knodes.shape
    nl = K + 1
    T = tree_depth(nl, 2)
    off = level_offsets(2, T)
    C = np.zeros((B, H, off[T + 1], D), dtype=np.float64)
    for n in range(K):
        d = (n + 1).bit_length() - 1
        i = n - ((1 << d) - 1)
        C[:, :, off[d + 1] + 2 * i] = knodes[:, :, n] / 2
        C[:, :, off[d + 1] + 2 * i + 1] = -knodes[:, :, n] / 2
    return C


def pool_compat(k: np.ndarray, leaf_block: int) -> np.ndarray:
    """Reference-layout summaries: in-order Haar of the block means, read in heap order.

    At ``leaf_block=1`` this is exactly what the adapters feed the reference
    (``baselines/treeattn_torch.py:63-74`` then ``_tree_mha.py:104``): node
    ``n`` uses in-order coefficient ``n+1``.
    """
    m = block_means(k, leaf_block)  # (B,H,NL,D)
    coef = np.moveaxis(haar_inorder(np.moveaxis(m, 2, 0)), 0, 2)  # (B,H,NL-1,D)
    return nodekeys_to_summaries(coef)


def pool_natural(k: np.ndarray, branching: int, leaf_block: int) -> np.ndarray:
    """Child summary of every non-root node: half the mean key of its subtree.

    For ``branching=2`` the left/right decision is ``sigmoid(q.(mL - mR)/2)``:
    the reference's logit with the Haar coefficient of the node's own subtree.
    """
    m = block_means(k, leaf_block)  # (B,H,NL,D)
    B, H, nl, D = m.shape
    T = tree_depth(nl, branching)
    off = level_offsets(branching, T)
    C = np.zeros((B, H, off[T + 1], D), dtype=np.float64)
    for lam in range(1, T + 1):
        nodes = branching**lam
        C[:, :, off[lam]:off[lam] + nodes] = m.reshape(B, H, nodes, nl // nodes, D).mean(axis=3) / 2
    return C


def pool_adjoint(dC: np.ndarray, L: int, branching: int, leaf_block: int, tree_mode: str) -> np.ndarray:
    """Transpose of the pooling map: ``dC (B,H,NS,D) -> dk (B,L,H,D)``."""
    B, H, NS, D = dC.shape
    nl = L // leaf_block
    T = tree_depth(nl, branching)
    off = level_offsets(branching, T)
    if tree_mode == "natural":
        dm = np.zeros((B, H, nl, D))
        for lam in range(1, T + 1):
            nodes = branching**lam
            per = nl // nodes
            blk = dC[:, :, off[lam]:off[lam] + nodes] / (2 * per)
            dm += np.repeat(blk, per, axis=2)
    elif tree_mode == "compat":
        dcoef = nodekeys_adjoint(dC)  # (B,H,NL-1,D)
        dm = np.moveaxis(haar_inorder_adjoint(np.moveaxis(dcoef, 2, 0)), 0, 2)
    else:
        raise ValueError(tree_mode)
    dk_blocks = dm / leaf_block  # (B,H,NL,D)
    return np.repeat(dk_blocks, leaf_block, axis=2).transpose(0, 2, 1, 3)


def nodekeys_adjoint(dC: np.ndarray) -> np.ndarray:
    """Transpose of ``nodekeys_to_summaries``: ``dk_n = (dC_left - dC_right)/2``."""
    B, H, NS, D = dC.shape
    K = NS // 2
    T = tree_depth(K + 1, 2)
    off = level_offsets(2, T)
    dk = np.zeros((B, H, K, D))
    for n in range(K):
        d = (n + 1).bit_length() - 1
        i = n - ((1 << d) - 1)
        dk[:, :, n] = (dC[:, :, off[d + 1] + 2 * i] - dC[:, :, off[d + 1] + 2 * i + 1]) / 2
    return dk


# --------------------------------------------------------------------------
# Reference structure restated (binary heap tree, one key per node)
# --------------------------------------------------------------------------


def _logsigmoid(x: np.ndarray) -> np.ndarray:
    return -np.logaddexp(0.0, -x)


def ref_sample_paths_non_causal(q: np.ndarray, knodes: np.ndarray, g: np.ndarray):
    """Restates ``_sample_paths_non_causal`` (``_tree_mha.py:78-122``).

    ``q``: (L,B,H,D); ``knodes``: (K,B,H,D) heap-indexed; ``g``: Gumbels
    (L,B,H,S,T,2).  Returns leaf indices (L,B,H,S) and log-probs.
    """
    L, B, H, D = q.shape
    K = knodes.shape[0]
    N = K + 1
    log_n = (N - 1).bit_length() if N > 1 else 0
    S = g.shape[3]
    nodes = np.zeros((L, B, H, S), dtype=np.int64)
    acc = np.zeros((L, B, H, S))
    bi = np.arange(B)[None, :, None, None]
    hi = np.arange(H)[None, None, :, None]
    for d in range(log_n):
        valid = nodes < K
        kd = knodes[np.clip(nodes, 0, K - 1), bi, hi]  # (L,B,H,S,D)
        dots = np.einsum("lbhd,lbhsd->lbhs", q, kd)
        logp = np.stack([_logsigmoid(dots), _logsigmoid(-dots)], axis=-1)
        dirs = np.argmax(logp + g[..., d, :], axis=-1)
        chosen = np.take_along_axis(logp, dirs[..., None], axis=-1)[..., 0]
        acc = acc + np.where(valid, chosen, -np.inf)
        nodes = 2 * nodes + 1 + dirs
    return nodes - K, acc


def ref_forward_non_causal(q: np.ndarray, knodes: np.ndarray, v: np.ndarray, g: np.ndarray):
    """Restates the stochastic non-causal ``hierarchical_attention``
    (``_tree_mha.py:391-407``): sample, mask, softmax over samples, gather, sum.

    Returns ``out (L,B,H,D)``, ``weights (L,B,H,S)``, leaf indices.
    """
    N = v.shape[0]
    idx, lp = ref_sample_paths_non_causal(q, knodes, g)
    valid = (idx >= 0) & (idx < N)
    lp = np.where(valid, lp, -np.inf)
    lp = lp - lp.max(axis=-1, keepdims=True)
    w = np.exp(lp)
    w = w / w.sum(axis=-1, keepdims=True)
    B, H = v.shape[1], v.shape[2]
    bi = np.arange(B)[None, :, None, None]
    hi = np.arange(H)[None, None, :, None]
    gathered = v[np.clip(idx, 0, N - 1), bi, hi]  # (L,B,H,S,D)
    out = np.einsum("lbhs,lbhsd->lbhd", w, gathered)
    return out, w, idx


# --------------------------------------------------------------------------
# Generalized semantics (what the HIP kernels implement)
# --------------------------------------------------------------------------


def _lse(x: np.ndarray, axis: int = -1) -> np.ndarray:
    m = np.max(x, axis=axis, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    with np.errstate(divide="ignore"):
        s = np.log(np.sum(np.exp(x - m_safe), axis=axis, keepdims=True)) + m_safe
    return np.squeeze(s, axis=axis)


def causal_boundary_logmass(logp_b: np.ndarray, digits: np.ndarray) -> np.ndarray:
    """Log allowed mass ``log A_d`` of each boundary-path node, bottom-up.

    ``logp_b`` (..., T, b): child log-probabilities at the boundary node of
    each depth; ``digits`` (..., T): the boundary leaf block's branch at each
    depth.  Children left of the boundary child are fully allowed (mass 1),
    the boundary child carries ``A_{d+1}``, children to its right none:
    ``A_d = sum_{j<j*} p_j + p_{j*} A_{d+1}``, ``A_T = 1``.  Sampling with
    ``p'_j = p_j A_child / A_d`` then draws exactly from the tree distribution
    restricted to allowed leaf blocks.  (The reference's causal sampler,
    ``_tree_mha.py:166-196,203-249``, instead uses leaf counts as the mass of
    fully-allowed subtrees and stops correcting once any (b,h,s) lane leaves
    the boundary; that coupled variant is not this function.)
    """
    T = digits.shape[-1]
    b = logp_b.shape[-1]
    out = np.zeros(digits.shape[:-1] + (T + 1,))
    jj = np.arange(b)
    for d in range(T - 1, -1, -1):
        js = digits[..., d][..., None]
        terms = np.where(jj < js, logp_b[..., d, :], -np.inf)
        terms = np.where(jj == js, logp_b[..., d, :] + out[..., d + 1][..., None], terms)
        out[..., d] = _lse(terms)
    return out


def tree_sample(
    q: np.ndarray,
    C: np.ndarray,
    branching: int,
    leaf_block: int,
    U: np.ndarray,
    causal: bool,
    max_logit: float = 1e3,
    N: int | None = None,
):
    """Per-query root-to-leaf sampling (generalizes ``_tree_mha.py:78-122``).

    ``q`` (B,L,H,D); ``C`` (B,H,NS,D) child summaries; ``U`` uniforms
    (B,L,H,S,T,b).  At depth ``d`` a sample at node ``i`` reads child logits
    ``x_j = clamp(q . C[off[d+1] + b*i + j], +-max_logit/2)``, takes
    ``logp = log_softmax(x)`` (plus the causal correction on the boundary
    path), and moves to ``argmax_j(logp'_j + g_j)`` (first maximum wins, as
    ``torch.argmax`` does).  Returns leaf block ids (B,L,H,S), accumulated
    log-probs (B,L,H,S) and the per-decision margins (B,L,H,S,T) between the
    best and second-best perturbed score, for parity gating.  ``N`` (leaf
    tokens, default ``L``) sets the causal alignment: query ``t`` sees tokens
    ``<= t + N - L``.
    """
    B, L, H, D = q.shape
    N = L if N is None else N
    b = branching
    nl = N // leaf_block
    T = tree_depth(nl, b)
    off = level_offsets(b, T)
    S = U.shape[3]
    idx = np.zeros((B, L, H, S), dtype=np.int64)
    lp = np.zeros((B, L, H, S))
    margins = np.full((B, L, H, S, max(T, 1)), np.inf)
    half = max_logit / 2
    jj = np.arange(b)
    for bb in range(B):
        for h in range(H):
            Q = q[bb, :, h].astype(np.float64)  # (L,D)
            Cb = C[bb, h]
            X = lambda cols: np.clip(path_logits(Q, Cb, cols), -half, half)  # noqa: E731
            node = np.zeros((L, S), dtype=np.int64)
            acc = np.zeros((L, S))
            if causal and T > 0:
                blk_t = (np.arange(L) + N - L) // leaf_block
                digits = np.stack([(blk_t // b ** (T - 1 - d)) % b for d in range(T)], axis=-1)
                bnode = np.stack([blk_t // b ** (T - d) for d in range(T)], axis=-1)  # (L,T)
                cols_b = np.asarray(off[1:T + 1])[None, :, None] + b * bnode[:, :, None] + jj  # (L,T,b)
                xb = X(cols_b)
                logp_b = xb - _lse(xb)[..., None]
                logA = causal_boundary_logmass(logp_b, digits)  # (L,T+1)
            for d in range(T):
                cols = off[d + 1] + b * node[..., None] + jj  # (L,S,b)
                x = X(cols)
                logp = x - _lse(x)[..., None]
                if causal:
                    on_b = node == bnode[:, d][:, None]  # (L,S)
                    js = digits[:, d][:, None, None]
                    corr = np.where(jj < js, 0.0, -np.inf)
                    corr = np.where(jj == js, logA[:, d + 1][:, None, None], corr)
                    corr = corr - logA[:, d][:, None, None]
                    logp = np.where(on_b[..., None], logp + corr, logp)
                score = logp + gumbel(U[bb, :, h, :, d, :])
                j = np.argmax(score, axis=-1)
                srt = np.sort(score, axis=-1)
                margins[bb, :, h, :, d] = srt[..., -1] - srt[..., -2] if b > 1 else np.inf
                acc += np.take_along_axis(logp, j[..., None], axis=-1)[..., 0]
                node = b * node + j
            idx[bb, :, h] = node
            lp[bb, :, h] = acc
    return idx, lp, margins


def path_logits(Q, C, cols):
    """``x[l, s, j] = Q[l] . C[cols[l, s, j]]`` for one (batch, head): ``Q`` (L, D),
    ``C`` (NS, D), ``cols`` (L, S, b).  From the dense ``Q C^T`` when it is small,
    else by gathering only the rows the paths visit (linear in L)."""
    L = Q.shape[0]
    if L * C.shape[0] <= 1 << 25:
        X = Q @ C.T
        return np.take_along_axis(X, cols.reshape(L, -1), axis=1).reshape(cols.shape)
    return np.matmul(C[cols.reshape(L, -1)], Q[:, :, None])[..., 0].reshape(cols.shape)


def path_logprobs(q, C, branching, num_leaf_blocks, idx, max_logit=1e3):
    """Uncorrected ``log P(leaf)`` of given sampled leaf blocks (B,L,H,S).

    In causal mode the sampler's accumulated log-probs differ from these by
    the per-query constant ``-log A_root``, which leaves ``softmax_s``
    (the weights) unchanged.
    """
    b = branching
    T = tree_depth(num_leaf_blocks, b)
    off = level_offsets(b, T)
    B, L, H, D = q.shape
    S = idx.shape[-1]
    half = max_logit / 2
    jj = np.arange(b)
    lp = np.zeros((B, L, H, S))
    for bb in range(B):
        for h in range(H):
            Q = q[bb, :, h].astype(np.float64)
            leaf = idx[bb, :, h]
            for d in range(T):
                node = leaf // b ** (T - d)
                js = (leaf // b ** (T - 1 - d)) % b
                cols = off[d + 1] + b * node[..., None] + jj  # (L, S, b)
                x = np.clip(path_logits(Q, C[bb, h], cols), -half, half)
                logp = x - _lse(x)[..., None]
                lp[bb, :, h] += np.take_along_axis(logp, js[..., None], axis=-1)[..., 0]
    return lp


def sample_weights(lp: np.ndarray) -> np.ndarray:
    """``softmax`` over samples (``_tree_mha.py:396-399``)."""
    m = lp.max(axis=-1, keepdims=True)
    e = np.exp(lp - m)
    return e / e.sum(axis=-1, keepdims=True)


def _leaf_gather(x64, idx_s, leaf_block):
    """``x[b, idx*LB + j, h]`` for one sample: (B,L,H) ids -> (B,L,H,LB,D)."""
    B, _, H, _ = x64.shape
    tok = idx_s[..., None] * leaf_block + np.arange(leaf_block)  # (B,L,H,LB)
    bi = np.arange(B)[:, None, None, None]
    hi = np.arange(H)[None, None, :, None]
    return x64[bi, tok, hi], tok


def leaf_attention(q, k, v, idx, leaf_block, causal, scale):
    """Per (query, sample): ``softmax(scale q.K_blk^T [mask]) V_blk``.

    Returns ``o_s`` (B,L,H,S,D) and the probabilities (B,L,H,S,LB).  At
    ``leaf_block=1`` this is ``v[idx]``, the reference's value gather
    (``_tree_mha.py:405``).  Causal: query ``t`` sees tokens
    ``<= t + N - L`` (bottom-right aligned).
    """
    B, L, H, D = q.shape
    N = v.shape[1]
    S = idx.shape[-1]
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    o = np.zeros((B, L, H, S, D))
    a_all = np.zeros((B, L, H, S, leaf_block))
    t = np.arange(L)[None, :, None, None] + (N - L)
    for s in range(S):
        Kg, tok = _leaf_gather(k64, idx[..., s], leaf_block)
        Vg, _ = _leaf_gather(v64, idx[..., s], leaf_block)
        z = scale * np.einsum("blhd,blhjd->blhj", q64, Kg)
        if causal:
            z = np.where(tok > t, -np.inf, z)
        z = z - z.max(axis=-1, keepdims=True)
        a = np.exp(z)
        a = a / a.sum(axis=-1, keepdims=True)
        a_all[..., s, :] = a
        o[..., s, :] = np.einsum("blhj,blhjd->blhd", a, Vg)
    return o, a_all


def tree_forward(q, k, v, C, branching, leaf_block, U, causal, scale=None, max_logit=1e3):
    """Full forward: ``o = sum_s w_s o_s`` with ``w = softmax_s(lp)``.

    Returns ``out (B,L,H,D)``, ``weights (B,L,H,S)``, leaf ids, log-probs and
    decision margins.
    """
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    idx, lp, margins = tree_sample(q, C, branching, leaf_block, U, causal, max_logit, N=v.shape[1])
    w = sample_weights(lp)
    o_s, _ = leaf_attention(q, k, v, idx, leaf_block, causal, scale)
    out = np.einsum("blhs,blhsd->blhd", w, o_s)
    return out, w, idx, lp, margins


def tree_backward(q, k, v, C, branching, leaf_block, idx, w, dout, causal, scale=None, max_logit=1e3):
    """Explicit gradient of ``<dout, out>`` given the sampled paths.

    Derivation (matches ``_autograd.py:744-858`` at ``LB=1``):
    ``delta_s = dout . o_s``; ``dlp_s = w_s (delta_s - sum w delta)``;
    leaf block: ``dP = w_s dout V^T``, ``dz = a (dP - w_s delta_s)``,
    ``dq += scale dz K``, ``dK += scale dz^T q``, ``dV += a^T w_s dout``;
    tree: at each depth ``dx_j = dlp_s (1[j=j*] - p_j)`` (zero where the logit
    is clamped), ``dq += sum_j dx_j C_j``, ``dC_j += dx_j q``.  The causal
    correction adds the same ``-log A_root`` to every sample of a query, so
    its gradient cancels exactly (``sum_s dlp_s = 0``).

    Returns ``dq (B,L,H,D)``, ``dC (B,H,NS,D)``, leaf ``dk``, ``dv``.
    """
    B, L, H, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    b = branching
    nl = v.shape[1] // leaf_block
    T = tree_depth(nl, b)
    off = level_offsets(b, T)
    S = idx.shape[-1]
    LB = leaf_block
    q64, k64, v64, g64 = (x.astype(np.float64) for x in (q, k, v, dout))
    o_s, a = leaf_attention(q, k, v, idx, leaf_block, causal, scale)
    delta = np.einsum("blhd,blhsd->blhs", g64, o_s)
    dlp = w * (delta - (w * delta).sum(axis=-1, keepdims=True))

    N = v.shape[1]
    dq = np.zeros((B, L, H, D))
    dk = np.zeros((B, N, H, D))
    dv = np.zeros((B, N, H, D))
    for s_ in range(S):
        Kg, tok = _leaf_gather(k64, idx[..., s_], LB)
        Vg, _ = _leaf_gather(v64, idx[..., s_], LB)
        ws = w[..., s_]
        dP = ws[..., None] * np.einsum("blhd,blhjd->blhj", g64, Vg)
        dz = a[..., s_, :] * (dP - (ws * delta[..., s_])[..., None])
        dq += scale * np.einsum("blhj,blhjd->blhd", dz, Kg)
        dKc = scale * dz[..., None] * q64[:, :, :, None, :]
        dVc = (a[..., s_, :] * ws[..., None])[..., None] * g64[:, :, :, None, :]
        bb = np.broadcast_to(np.arange(B)[:, None, None, None], tok.shape)
        hh = np.broadcast_to(np.arange(H)[None, None, :, None], tok.shape)
        np.add.at(dk, (bb, tok, hh), dKc)
        np.add.at(dv, (bb, tok, hh), dVc)

    half = max_logit / 2
    dC = np.zeros(C.shape)
    jj = np.arange(b)
    for b_ in range(B):
        for h in range(H):
            Q = q64[b_, :, h]
            Xr = Q @ C[b_, h].T
            X = np.clip(Xr, -half, half)
            live = (Xr >= -half) & (Xr <= half)
            leaf = idx[b_, :, h]  # (L,S)
            for d in range(T):
                node = leaf // b ** (T - d)
                jstar = (leaf // b ** (T - 1 - d)) % b
                cols = off[d + 1] + b * node[..., None] + jj  # (L,S,b)
                x = np.take_along_axis(X, cols.reshape(L, -1), axis=1).reshape(L, S, b)
                lv = np.take_along_axis(live, cols.reshape(L, -1), axis=1).reshape(L, S, b)
                p = np.exp(x - _lse(x)[..., None])
                dx = dlp[b_, :, h][..., None] * ((jj == jstar[..., None]) - p) * lv
                dq[b_, :, h] += np.einsum("lsj,lsjd->ld", dx, C[b_, h][cols])
                np.add.at(dC[b_, h], cols.reshape(-1), (dx[..., None] * Q[:, None, None, :]).reshape(-1, D))
    return dq, dC, dk, dv


def head_fwd_bwd(q, k, v, dout, C, branching, leaf_block, idx, causal, scale, max_logit=1e3):
    """``tree_forward`` + ``tree_backward`` of ONE (batch, head) on given paths,
    organized by leaf block so that full-size heads run in seconds (child
    logits only along the sampled paths: linear in L for any tree).

    Same mathematics as ``leaf_attention`` / ``sample_weights(path_logprobs)``
    / ``tree_backward`` (``_tree_mha.py:396-407``, ``_autograd.py:744-858``),
    but every (query, sample) pair of a leaf block is processed as one matrix
    product against that block's keys and values, and the child-logit
    gradient is a sparse ``(L, NS)`` matrix ``G`` with ``dq += G C`` and
    ``dC = G^T q``.  Pinned against those functions in
    ``tests/test_oracle.py::test_head_fwd_bwd_matches_explicit``.

    ``q``, ``dout`` (L, D); ``k``, ``v`` (N, D); ``C`` (NS, D) child summaries;
    ``idx`` (L, S) leaf blocks.  Returns a dict with ``out`` (L, D),
    ``weights`` (L, S), ``dq`` (L, D), ``dC`` (NS, D), ``dk_leaf``, ``dv`` (N, D).
    """
    q64, k64, v64, g64, C64 = (np.asarray(x, dtype=np.float64) for x in (q, k, v, dout, C))
    L, D = q64.shape
    N = v64.shape[0]
    S = idx.shape[1]
    b, LB = branching, leaf_block
    nl = N // LB
    T = tree_depth(nl, b)
    off = level_offsets(b, T)
    lp = path_logprobs(q64[None, :, None], C64[None, None], b, nl, idx[None, :, None], max_logit)[0, :, 0]
    w = sample_weights(lp)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    starts = np.searchsorted(flat[order], np.arange(nl + 1))
    pos = np.arange(L) + (N - L)

    def block_pairs(beta):
        pr = order[starts[beta]:starts[beta + 1]]
        l_p, s_p = pr // S, pr % S
        Kb, Vb = k64[beta * LB:(beta + 1) * LB], v64[beta * LB:(beta + 1) * LB]
        z = scale * (q64[l_p] @ Kb.T)
        if causal:
            z = np.where(beta * LB + np.arange(LB)[None, :] > pos[l_p][:, None], -np.inf, z)
        z = z - z.max(axis=1, keepdims=True)
        a = np.exp(z)
        a /= a.sum(axis=1, keepdims=True)
        return l_p, s_p, Kb, Vb, a

    o_pair = np.zeros((L, S, D))
    for beta in range(nl):
        l_p, s_p, _, Vb, a = block_pairs(beta)
        o_pair[l_p, s_p] = a @ Vb
    out = np.einsum("ls,lsd->ld", w, o_pair)
    delta = np.einsum("ld,lsd->ls", g64, o_pair)
    dlp = w * (delta - (w * delta).sum(axis=1, keepdims=True))

    dq_pair = np.zeros((L, S, D))
    dk = np.zeros((N, D))
    dv = np.zeros((N, D))
    for beta in range(nl):
        l_p, s_p, Kb, Vb, a = block_pairs(beta)
        ws = w[l_p, s_p]
        Gl = g64[l_p]
        dz = a * (ws[:, None] * (Gl @ Vb.T) - (ws * delta[l_p, s_p])[:, None])
        dq_pair[l_p, s_p] = scale * (dz @ Kb)
        dk[beta * LB:(beta + 1) * LB] = scale * (dz.T @ q64[l_p])
        dv[beta * LB:(beta + 1) * LB] = (a * ws[:, None]).T @ Gl
    dq = dq_pair.sum(axis=1)

    # child logits only along the sampled paths, so trees with many nodes per
    # level stay linear in L; G (queries x summary rows) is a sparse matrix
    from scipy import sparse

    half = max_logit / 2
    jj = np.arange(b)
    rows = np.broadcast_to(np.arange(L)[:, None, None], (L, S, b))
    gr, gc, gv = [], [], []
    for d in range(T):
        node = idx // b ** (T - d)
        jstar = (idx // b ** (T - 1 - d)) % b
        cols = off[d + 1] + b * node[..., None] + jj  # (L, S, b)
        xr = path_logits(q64, C64, cols)
        x = np.clip(xr, -half, half)
        p = np.exp(x - _lse(x)[..., None])
        lv = (xr >= -half) & (xr <= half)
        dx = dlp[..., None] * ((jj == jstar[..., None]) - p) * lv
        gr.append(rows.reshape(-1))
        gc.append(cols.reshape(-1))
        gv.append(dx.reshape(-1))
    G = sparse.coo_matrix((np.concatenate(gv), (np.concatenate(gr), np.concatenate(gc))),
                          shape=(L, C64.shape[0])).tocsr()  # duplicate entries add
    dq += G @ C64
    dC = np.asarray(G.T @ q64)
    return dict(out=out, weights=w, lp=lp, dq=dq, dC=dC, dk_leaf=dk, dv=dv)


def summaries(k, branching, leaf_block, tree_mode):
    """Child summaries for ``tree_mode`` in {"natural", "compat"}."""
    if tree_mode == "natural":
        return pool_natural(k, branching, leaf_block)
    if tree_mode == "compat":
        if branching != 2:
            raise ValueError("compat summaries need branching=2")
        return pool_compat(k, leaf_block)
    raise ValueError(f"unknown tree_mode {tree_mode!r}")


def attention_fwd_bwd(q, k, v, dout, branching, leaf_block, U, causal, tree_mode,
                      scale=None, max_logit=1e3):
    """Adapter-level forward + backward on bshd tensors (float64 results).

    Returns a dict with ``out, weights, idx, lp, margins, dq, dk, dv``.
    """
    B, L, H, D = q.shape
    C = summaries(k.astype(np.float64), branching, leaf_block, tree_mode)
    out, w, idx, lp, margins = tree_forward(q, k, v, C, branching, leaf_block, U, causal, scale, max_logit)
    res = dict(out=out, weights=w, idx=idx, lp=lp, margins=margins)
    if dout is not None:
        dq, dC, dk_leaf, dv = tree_backward(q, k, v, C, branching, leaf_block, idx, w, dout, causal,
                                            scale, max_logit)
        dk = dk_leaf + pool_adjoint(dC, k.shape[1], branching, leaf_block, tree_mode)
        res.update(dq=dq, dk=dk, dv=dv, dC=dC)
    return res


# --------------------------------------------------------------------------
# Packed path record (_autograd.py:68-90,179-216).
# --------------------------------------------------------------------------


def path_bytes(num_leaf_blocks: int) -> int:
    """Bytes per packed path: ``_path_bit_bytes`` (``_autograd.py:68-70``)."""
    return (max(int(num_leaf_blocks).bit_length() - 1, 0) + 7) // 8


def pack_paths(idx: np.ndarray, num_leaf_blocks: int) -> np.ndarray:
    """Leaf block ids ``(..., S)`` -> packed bits ``(..., S, path_bytes)`` uint8.

    Bit ``p`` of a path (``p = 0`` at the root) sits in byte ``p // 8`` at bit
    ``p % 8`` (``_autograd.py:214-216``); the path's bits are the id's, most
    significant first (for a binary heap, bit ``d`` is the direction taken at
    depth ``d``; in a ``b``-ary tree each level's digit takes ``log2 b`` bits).
    """
    nbits = int(num_leaf_blocks).bit_length() - 1
    idx = np.asarray(idx, dtype=np.int64)
    out = np.zeros(idx.shape + (path_bytes(num_leaf_blocks),), dtype=np.uint8)
    for p in range(nbits):
        bit = (idx >> (nbits - 1 - p)) & 1
        out[..., p // 8] |= (bit << (p % 8)).astype(np.uint8)
    return out


def unpack_paths(packed: np.ndarray, num_leaf_blocks: int) -> np.ndarray:
    """Inverse of ``pack_paths``: ``(..., bytes)`` uint8 -> leaf block ids (int64)."""
    nbits = int(num_leaf_blocks).bit_length() - 1
    packed = np.asarray(packed, dtype=np.int64)
    idx = np.zeros(packed.shape[:-1], dtype=np.int64)
    for p in range(nbits):
        idx |= ((packed[..., p // 8] >> (p % 8)) & 1) << (nbits - 1 - p)
    return idx


def heap_walk(directions: np.ndarray) -> np.ndarray:
    """The reference's root-to-leaf walk: per depth ``node <- 2 node + 1 + dir``,
    leaf ``= node - K`` with ``K = 2^T - 1`` (``_autograd.py:219,312-315``)."""
    T = directions.shape[-1]
    node = np.zeros(directions.shape[:-1], dtype=np.int64)
    for d in range(T):
        node = 2 * node + 1 + directions[..., d].astype(np.int64)
    return node - (2 ** T - 1)
