"""Timed CPU baseline: the reference's CPU path restated in torch -- TEST / BASELINE
INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg import this module: it is
the CPU path the GPU kernels are timed against, never part of the product
(``treeattention_amd`` does not import it).

It follows the structure of treeattn-torch's stochastic op
(``packages/treeattn-torch/src/treeattn_torch/_tree_mha.py:78-122,396-407``) on
float32 CPU tensors with every host core, generalized to the branching ``b``
and leaf block ``LB`` of the benchmark configs exactly as the HIP kernels are:

* summaries (``_treeattn_common.py:54-86`` for ``compat``; per-level child means
  for ``natural``);
* per depth, for a block of queries at a time (the reference streams query
  blocks, ``_autograd.py:223-257``): gather the children's summaries of every
  sample's node (``_gather_keys_by_index``, ``_tree_mha.py:45-75``), dot with
  the query, clamp (``_autograd.py:202``), log-softmax, the exact causal
  correction on the boundary path, Gumbel noise from the explicit uniforms,
  ``argmax``, accumulate the chosen log-probability (``:99-119``);
* ``softmax`` over samples (``:399``) and per (query, sample) the leaf block's
  gathered keys and values, ``softmax(scale q K^T [mask]) V`` (at ``LB = 1`` the
  value gather of ``:405``), summed with the weights (``:407``);
* backward: the explicit streaming form of ``_autograd.py:706-860`` (per query
  block: ``delta = dout . o_s``, ``dlp = w (delta - sum w delta)``, leaf
  gradients, per depth ``dx = dlp (1[j = j*] - p)``, ``dq += dx C``,
  ``dC[node] += dx q`` by ``index_add_``), then the summaries' adjoint.

Pinned against ``oracle.tree_oracle`` (float64) in ``tests/test_cpu_path.py``.
"""

from __future__ import annotations

import math

import torch

from . import tree_oracle as O


def _gumbel(u: torch.Tensor) -> torch.Tensor:
    return -torch.log(-torch.log(u))


def summaries(k: torch.Tensor, b: int, LB: int, tree_mode: str) -> torch.Tensor:
    """``k (N, H, D)`` -> child summaries ``(H, NS, D)`` (levels 1..T, unpadded, as
    ``oracle.tree_oracle.level_offsets``)."""
    N, H, D = k.shape
    nl = N // LB
    T = O.tree_depth(nl, b)
    m = k.reshape(nl, LB, H, D).mean(dim=1)  # (NL, H, D) leaf-block means
    if tree_mode == "natural":
        lv = [m.reshape(b**lam, nl // b**lam, H, D).mean(dim=1) / 2 for lam in range(1, T + 1)]
        return torch.cat(lv, dim=0).permute(1, 0, 2).contiguous()
    if tree_mode != "compat" or b != 2:
        raise ValueError("compat summaries are binary")
    out = m.clone()  # in-order Haar coefficients of the block means (_treeattn_common.py:65-86)
    for level in range(T):
        step = 1 << level
        base = torch.arange(nl >> (level + 1)) * (2 * step)
        a_, c_ = out[base], out[base + step]
        out[base] = (a_ + c_) / 2
        out[base + step] = (a_ - c_) / 2
    kn = out[1:]  # read in heap order: node n uses coefficient n + 1
    lv = []
    for lam in range(1, T + 1):
        nodes = kn[(1 << (lam - 1)) - 1:(1 << lam) - 1]  # (2^(lam-1), H, D)
        lv.append(torch.stack([nodes / 2, -nodes / 2], dim=1).reshape(2 << (lam - 1), H, D))
    return torch.cat(lv, dim=0).permute(1, 0, 2).contiguous()


def summaries_adjoint(dC: torch.Tensor, N: int, b: int, LB: int, tree_mode: str) -> torch.Tensor:
    """Transpose of ``summaries``: ``dC (H, NS, D)`` -> ``dk (N, H, D)``."""
    H, NS, D = dC.shape
    nl = N // LB
    T = O.tree_depth(nl, b)
    off = O.level_offsets(b, T)
    if tree_mode == "natural":
        dm = torch.zeros(nl, H, D)
        for lam in range(1, T + 1):
            nodes, per = b**lam, nl // b**lam
            blk = dC[:, off[lam]:off[lam] + nodes].permute(1, 0, 2) / (2 * per)  # (nodes, H, D)
            dm += blk.repeat_interleave(per, dim=0)
    else:
        dcoef = torch.zeros(nl, H, D)
        for lam in range(1, T + 1):
            rows = dC[:, off[lam]:off[lam] + (2 << (lam - 1))].permute(1, 0, 2).reshape(-1, 2, H, D)
            dcoef[1 << (lam - 1):1 << lam] = (rows[:, 0] - rows[:, 1]) / 2
        for level in reversed(range(T)):
            step = 1 << level
            base = torch.arange(nl >> (level + 1)) * (2 * step)
            da, dd = dcoef[base].clone(), dcoef[base + step].clone()
            dcoef[base] = (da + dd) / 2
            dcoef[base + step] = (da - dd) / 2
        dm = dcoef
    return (dm / LB).repeat_interleave(LB, dim=0)


class Problem:
    """One batch element: ``q``/``dout`` (Lq, H, D), ``k``/``v`` (N, H, D), uniforms
    ``U`` (Lq, H, S, T, b) and ``pos`` (Lq,): the last token each query may see
    when causal (bottom-right aligned: query ``t`` of ``L`` sees ``t + N - L``)."""

    def __init__(self, q, k, v, U, pos, b, LB, causal, tree_mode, scale=None, max_logit=1e3, qblock=64):
        self.q, self.k, self.v = (x.float().contiguous() for x in (q, k, v))
        self.U = torch.as_tensor(U).float()
        self.pos = torch.as_tensor(pos).long()
        self.b, self.LB, self.causal, self.mode = b, LB, causal, tree_mode
        self.N = self.k.shape[0]
        self.nl = self.N // LB
        self.T = O.tree_depth(self.nl, b)
        self.off = O.level_offsets(b, self.T)
        self.S = self.U.shape[2]
        self.scale = scale if scale is not None else 1.0 / math.sqrt(self.q.shape[-1])
        self.half = max_logit / 2
        self.qblock = qblock

    def _child_rows(self, C, node, d):
        """Gathered child summaries of each sample's node at depth d: (lq, H, S, b, D)."""
        H = C.shape[0]
        cols = self.off[d + 1] + self.b * node.unsqueeze(-1) + torch.arange(self.b)  # (lq, H, S, b)
        hh = torch.arange(H).view(1, H, 1, 1)
        return C[hh, cols], cols

    def _boundary_logmass(self, C, qb, pb):
        """Exact causal: log allowed mass at each boundary-path node, (lq, H, T + 1)."""
        b, T = self.b, self.T
        bl = pb // self.LB  # (lq,) boundary leaf block
        H = C.shape[0]
        digits = torch.stack([(bl // b ** (T - 1 - d)) % b for d in range(T)], dim=-1)  # (lq, T)
        bnode = torch.stack([bl // b ** (T - d) for d in range(T)], dim=-1)
        logA = torch.zeros(qb.shape[0], H, T + 1)
        jj = torch.arange(b)
        for d in range(T - 1, -1, -1):
            cols = self.off[d + 1] + b * bnode[:, d].view(-1, 1, 1) + jj  # (lq, 1, b)
            Cg = C[torch.arange(H).view(1, H, 1), cols.expand(-1, H, -1)]  # (lq, H, b, D)
            x = (qb.unsqueeze(2) * Cg).sum(-1).clamp(-self.half, self.half)
            lp = torch.log_softmax(x, dim=-1)
            js = digits[:, d].view(-1, 1, 1)
            terms = torch.where(jj < js, lp, torch.full_like(lp, -math.inf))
            terms = torch.where(jj == js, lp + logA[:, :, d + 1:d + 2], terms)
            logA[:, :, d] = torch.logsumexp(terms, dim=-1)
        return logA, digits, bnode

    def forward(self, C, forced=None):
        """Returns ``idx (Lq, H, S)``, ``w``, ``out (Lq, H, D)``."""
        Lq, H, D = self.q.shape
        b, S = self.b, self.S
        idx = torch.empty(Lq, H, S, dtype=torch.long)
        w = torch.empty(Lq, H, S)
        out = torch.empty(Lq, H, D)
        g_all = _gumbel(self.U)
        for l0 in range(0, Lq, self.qblock):
            sl = slice(l0, min(Lq, l0 + self.qblock))
            qb, pb = self.q[sl], self.pos[sl]
            lq = qb.shape[0]
            node = torch.zeros(lq, H, S, dtype=torch.long)
            acc = torch.zeros(lq, H, S)
            if self.causal:
                logA, digits, bnode = self._boundary_logmass(C, qb, pb)
            for d in range(self.T):
                Cg, _ = self._child_rows(C, node, d)
                x = (qb.view(lq, H, 1, 1, D) * Cg).sum(-1).clamp(-self.half, self.half)  # (lq, H, S, b)
                lp = torch.log_softmax(x, dim=-1)
                if self.causal:
                    on_b = node == bnode[:, d].view(-1, 1, 1)
                    jj = torch.arange(b)
                    js = digits[:, d].view(-1, 1, 1, 1)
                    corr = torch.where(jj < js, 0.0, -math.inf)
                    corr = torch.where(jj == js, logA[:, :, d + 1].view(lq, H, 1, 1), corr)
                    corr = corr - logA[:, :, d].view(lq, H, 1, 1)
                    lp = torch.where(on_b.unsqueeze(-1), lp + corr, lp)
                score = lp + g_all[sl, :, :, d, :]
                j = torch.argmax(score, dim=-1) if forced is None else (forced[sl] // b ** (self.T - 1 - d)) % b
                acc += torch.gather(lp, -1, j.unsqueeze(-1)).squeeze(-1)
                node = b * node + j
            idx[sl] = node
            wb = torch.softmax(acc, dim=-1)
            w[sl] = wb
            o_s, _ = self._leaf(qb, pb, node)
            out[sl] = (wb.unsqueeze(-1) * o_s).sum(2)
        return idx, w, out

    def _leaf(self, qb, pb, node):
        """Per (query, sample) ``softmax(scale q K_blk^T [mask]) V_blk``: (lq, H, S, D), probs."""
        lq, H, D = qb.shape
        tok = node.unsqueeze(-1) * self.LB + torch.arange(self.LB)  # (lq, H, S, LB)
        hh = torch.arange(H).view(1, H, 1, 1)
        Kg, Vg = self.k[tok, hh], self.v[tok, hh]  # (lq, H, S, LB, D)
        z = self.scale * (qb.view(lq, H, 1, 1, D) * Kg).sum(-1)
        if self.causal:
            z = z.masked_fill(tok > pb.view(-1, 1, 1, 1), -math.inf)
        a = torch.softmax(z, dim=-1)
        return (a.unsqueeze(-1) * Vg).sum(3), (a, tok, Kg, Vg)

    def backward(self, C, idx, w, dout):
        """Returns ``dq (Lq, H, D)``, ``dk (N, H, D)``, ``dv (N, H, D)``."""
        Lq, H, D = self.q.shape
        b, LB, S = self.b, self.LB, self.S
        dout = dout.float()
        dq = torch.zeros(Lq, H, D)
        dk = torch.zeros(self.N * H, D)
        dv = torch.zeros(self.N * H, D)
        dC = torch.zeros(H * C.shape[1], D)
        NS = C.shape[1]
        for l0 in range(0, Lq, self.qblock):
            sl = slice(l0, min(Lq, l0 + self.qblock))
            qb, pb, gb, nb, wb = self.q[sl], self.pos[sl], dout[sl], idx[sl], w[sl]
            lq = qb.shape[0]
            o_s, (a, tok, Kg, Vg) = self._leaf(qb, pb, nb)
            delta = (gb.unsqueeze(2) * o_s).sum(-1)  # (lq, H, S)
            dlp = wb * (delta - (wb * delta).sum(-1, keepdim=True))
            dP = wb.unsqueeze(-1) * (gb.view(lq, H, 1, 1, D) * Vg).sum(-1)  # (lq, H, S, LB)
            dz = a * (dP - (wb * delta).unsqueeze(-1))
            dq[sl] += self.scale * (dz.unsqueeze(-1) * Kg).sum((2, 3))
            rows = (tok * H + torch.arange(H).view(1, H, 1, 1)).reshape(-1)
            dk.index_add_(0, rows, (self.scale * dz.unsqueeze(-1) * qb.view(lq, H, 1, 1, D)).reshape(-1, D))
            dv.index_add_(0, rows, ((a * wb.unsqueeze(-1)).unsqueeze(-1) * gb.view(lq, H, 1, 1, D)).reshape(-1, D))
            node = torch.zeros(lq, H, S, dtype=torch.long)
            for d in range(self.T):
                Cg, cols = self._child_rows(C, node, d)
                xr = (qb.view(lq, H, 1, 1, D) * Cg).sum(-1)
                live = (xr >= -self.half) & (xr <= self.half)
                p = torch.softmax(xr.clamp(-self.half, self.half), dim=-1)
                j = (nb // b ** (self.T - 1 - d)) % b
                onehot = torch.nn.functional.one_hot(j, b).float()
                dx = dlp.unsqueeze(-1) * (onehot - p) * live
                dq[sl] += (dx.unsqueeze(-1) * Cg).sum((2, 3))
                crow = (torch.arange(H).view(1, H, 1, 1) * NS + cols).reshape(-1)
                dC.index_add_(0, crow, (dx.unsqueeze(-1) * qb.view(lq, H, 1, 1, D)).reshape(-1, D))
                node = b * node + j
        dk = dk.view(self.N, H, D) + summaries_adjoint(dC.view(H, NS, D), self.N, b, LB, self.mode)
        return dq, dk, dv.view(self.N, H, D)
