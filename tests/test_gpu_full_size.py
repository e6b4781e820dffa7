"""GPU checks at BASELINE.json's full sizes (C2-C5), where the float64 oracle
cannot run the whole problem:

* complete-head parity (C2, C3, C5): heads are independent, so one whole
  (batch, head) of the full problem -- all L queries and all N keys -- is
  checked against the oracle: leaves, weights, out, dq, dk and dv;
* parity on a query subset: the last 64 queries of the first and the last
  (batch, head) -- with bottom-right causal alignment a suffix keeps its
  positions -- against the oracle with the same in-kernel uniforms (Philox
  words computed for exactly those samples): sampled leaf blocks equal where
  every decision's margin exceeds 1e-3, weights, output rows and dq rows
  within 2e-2 on the GPU's own paths;
* size-independent identities over the whole problem: weights are a softmax
  over samples (non-negative, summing to one), every sampled block is
  reachable (causal), sum_n dv_n = sum_l dout_l per (batch, head) (each
  sample's leaf softmax and the sample weights sum to one), and
  sum_n dk_n = 0 per (batch, head) (shifting every key of a head by one vector
  changes neither a leaf block's softmax nor any node's child softmax).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import tree_oracle as O

pytestmark = pytest.mark.gpu

# name: B, L, H, D, dtype, branching, leaf block, samples, causal, input kind
FULL = {
    "C2": (4, 4096, 16, 64, torch.bfloat16, 2, 64, 8, False, "normal"),
    "C3": (2, 16384, 16, 128, torch.bfloat16, 4, 64, 16, True, "normal"),
    "C4": (1, 131072, 8, 128, torch.bfloat16, 2, 128, 16, False, "scaled"),
    "C5-D32": (8, 8192, 32, 32, torch.float16, 2, 32, 8, True, "skewed"),
    "C5-D96": (8, 8192, 32, 96, torch.float16, 2, 32, 8, True, "skewed"),
}
SUB = 64


def inputs(B, L, H, D, dtype, kind):
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v, do = (torch.randn(B, L, H, D, device="cuda", generator=g) for _ in range(4))
    if kind == "scaled":
        q, k, v = (x / math.sqrt(D) for x in (q, k, v))
    elif kind == "skewed":  # Student-t(3) keys, queries with a shared direction x3
        chi = sum(torch.randn(B, L, H, 1, device="cuda", generator=g) ** 2 for _ in range(3)) / 3
        k = k / chi.sqrt()
        u = torch.randn(D, device="cuda", generator=g)
        q = q + 3 * u / u.norm()
    return [x.to(dtype) for x in (q, k, v, do)]


uniforms_at = O.uniforms_at  # the generator's uniforms at flat indices of the (B, L, H, S, T, b) tensor


def rel(x, y):
    return float(np.linalg.norm(x - y) / max(np.linalg.norm(y), 1e-30))


@pytest.mark.parametrize("name", sorted(FULL))
def test_full_size(name):
    from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

    B, L, H, D, dtype, b, LB, S, causal, kind = FULL[name]
    mode = "natural" if b != 2 else "compat"
    print(f"[case] full size {name}: B={B} L={L} H={H} D={D} {dtype} b={b} LB={LB} S={S} causal={causal}", flush=True)
    q, k, v, do = inputs(B, L, H, D, dtype, kind)
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode=mode, causal=causal, seed=0)
    out, w, rec = tree_forward(q, k, v, opts)
    leaves_t, _ = record_views(q, k, v, opts, rec)
    dq, dk, dv = tree_backward(q, k, v, w, rec, do, opts)
    torch.cuda.synchronize()
    NL = L // LB
    T = round(math.log(NL, b))

    # identities over the whole problem
    for t in (out, dq, dk, dv):
        assert torch.isfinite(t.float()).all()
    assert (w >= 0).all() and (w.sum(-1) - 1).abs().max().item() < 1e-5
    assert int(leaves_t.min()) >= 0 and int(leaves_t.max()) < NL
    if causal:
        blk = (torch.arange(L, device="cuda") // LB).view(1, L, 1, 1)
        assert (leaves_t <= blk).all()
    sdv, sdo = dv.float().sum(1), do.float().sum(1)  # (B, H, D)
    assert rel(sdv.cpu().numpy(), sdo.cpu().numpy()) < 2e-2
    dkf = dk.float()
    shift = dkf.sum(1).norm(dim=-1)                                      # |sum_n dk_n| per (b, h)
    scale_ = dkf.pow(2).sum((1, 3)).sqrt()                               # sqrt(N) * rms row norm
    assert (shift / scale_).max().item() < 2e-2, (shift / scale_).max().item()

    # parity on the last SUB queries of the first and the last (batch, head)
    sc = 1.0 / math.sqrt(D)
    lsub = np.arange(L - SUB, L)
    for bb, h in ((0, 0), (B - 1, H - 1)):
        f64 = lambda t: t[bb:bb + 1, :, h:h + 1].float().cpu().numpy().astype(np.float64)
        kq, vq = f64(k), f64(v)
        qs, dos = f64(q)[:, -SUB:], f64(do)[:, -SUB:]
        C = O.summaries(kq, b, LB, mode)
        s_, t_, j_ = np.meshgrid(np.arange(S), np.arange(T), np.arange(b), indexing="ij")
        flat = (((((bb * L + lsub[:, None, None, None]) * H + h) * S + s_[None]) * T + t_[None]) * b + j_[None])
        U = uniforms_at(0, flat.reshape(-1)).reshape(1, SUB, 1, S, T, b)
        idx_o, _, margins = O.tree_sample(qs, C, b, LB, U, causal, N=L)
        lv = leaves_t[bb:bb + 1, -SUB:, h:h + 1].cpu().numpy().astype(np.int64)
        clean = margins.min(axis=-1) > 1e-3
        assert not ((lv != idx_o) & clean).any(), f"{int(((lv != idx_o) & clean).sum())} clean samples differ"
        assert clean.mean() > 0.9
        w_ref = O.sample_weights(O.path_logprobs(qs, C, b, NL, lv))
        o_s, _ = O.leaf_attention(qs, kq, vq, lv, LB, causal, sc)
        out_ref = np.einsum("blhs,blhsd->blhd", w_ref, o_s)
        assert rel(w[bb:bb + 1, -SUB:, h:h + 1].cpu().numpy(), w_ref) < 1e-4
        assert rel(f64(out)[:, -SUB:], out_ref) < 2e-2
        dq_o, _, _, _ = O.tree_backward(qs, kq, vq, C, b, LB, lv, w_ref, dos, causal, sc)
        r = rel(f64(dq)[:, -SUB:], dq_o)
        print(f"  (b={bb}, h={h}) clean {clean.mean():.3f}, dq rel err {r:.3g}", flush=True)
        assert r < 2e-2


# Deterministic (exact) mode through the attn-bench adapter at the C2 and C3
# shapes: the streaming kernels, no (L, N) buffer.
DET_FULL = {
    "C2-shape": (4, 4096, 16, 64, False),
    "C3-shape": (2, 16384, 16, 128, True),
}


@pytest.mark.parametrize("name", sorted(DET_FULL))
def test_deterministic_adapter_full_size(name, monkeypatch):
    """Full-size adapter path with TREEATTN_NUM_SAMPLES unset: the identities
    sum_n dv_n = sum_l dout_l (each query's exact weights sum to one) and
    sum_n dk_n = 0 (the Haar node keys drop every shift of the keys) per
    (batch, head), and out / dq rows of the last 64 queries of two heads
    against the float64 restatement (``ref_torch.leaf_logprobs``, softmax over
    the visible leaves when causal, autograd for dq)."""
    import treeattention_amd as ta
    from oracle import ref_torch as R

    monkeypatch.delenv("TREEATTN_NUM_SAMPLES", raising=False)
    for var in ("TREEATTN_BRANCHING", "TREEATTN_LEAF_BLOCK", "TREEATTN_TREE_MODE"):
        monkeypatch.delenv(var, raising=False)
    B, L, H, D, causal = DET_FULL[name]
    print(f"[case] deterministic adapter full size {name}: B={B} L={L} H={H} D={D} causal={causal}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v, do = (torch.randn(B, L, H, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(4))
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = ta.attn_fn(qg, kg, vg, causal, None)
    out.backward(do)
    torch.cuda.synchronize()
    for t in (out, qg.grad, kg.grad, vg.grad):
        assert torch.isfinite(t.float()).all()
    assert rel(vg.grad.float().sum(1).cpu().numpy(), do.float().sum(1).cpu().numpy()) < 2e-2
    dkf = kg.grad.float()
    assert (dkf.sum(1).norm(dim=-1) / dkf.pow(2).sum((1, 3)).sqrt()).max().item() < 2e-2

    for bb, h in ((0, 0), (B - 1, H - 1)):
        to64 = lambda t: t[bb:bb + 1, :, h:h + 1].double().cpu().permute(1, 0, 2, 3)  # (L, 1, 1, D)
        kq, vq = to64(k), to64(v)
        kn = torch.from_numpy(O.haar_inorder(kq.numpy()))  # (L-1, 1, 1, D) heap-ordered node keys
        qs = to64(q)[-SUB:].clone().requires_grad_(True)
        lpp = R.leaf_logprobs(qs, kn)  # (SUB, 1, 1, L)
        if causal:
            vis = torch.arange(L).view(1, L) <= torch.arange(L - SUB, L).view(SUB, 1)
            w = torch.softmax(lpp.masked_fill(~vis[:, None, None, :], float("-inf")), dim=-1)
        else:
            w = torch.exp(lpp)
        o_ref = torch.einsum("lbhn,nbhd->lbhd", w, vq)
        o_ref.backward(to64(do)[-SUB:])
        assert rel(to64(out.detach())[-SUB:].numpy(), o_ref.detach().numpy()) < 2e-2
        r = rel(to64(qg.grad)[-SUB:].numpy(), qs.grad.numpy())
        print(f"  (b={bb}, h={h}) dq rel err {r:.3g}", flush=True)
        assert r < 2e-2


@pytest.mark.parametrize("name", ["C2", "C3", "C5-D32", "C5-D96"])
def test_full_size_complete_head(name):
    """One complete (batch, head) at the full BASELINE size against the oracle:
    heads are independent, so the last (batch, head) of the full problem is
    exactly a one-head problem.  Sampled leaf blocks of all L queries equal the
    oracle's wherever every decision margin exceeds 1e-3; weights, out, dq, dk
    and dv of the whole head (every query, every key) within 2e-2 on the GPU's
    own paths (``O.head_fwd_bwd``, pinned against the explicit oracle)."""
    from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

    B, L, H, D, dtype, b, LB, S, causal, kind = FULL[name]
    mode = "natural" if b != 2 else "compat"
    print(f"[case] complete head {name}: B={B} L={L} H={H} D={D} {dtype} b={b} LB={LB} S={S} causal={causal}",
          flush=True)
    q, k, v, do = inputs(B, L, H, D, dtype, kind)
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode=mode, causal=causal, seed=0)
    out, w, rec = tree_forward(q, k, v, opts)
    leaves_t, _ = record_views(q, k, v, opts, rec)
    dq, dk, dv = tree_backward(q, k, v, w, rec, do, opts)
    torch.cuda.synchronize()
    bb, h = B - 1, H - 1
    one = lambda t: t[bb, :, h].float().cpu().numpy().astype(np.float64)  # noqa: E731  (L, D)
    qh, kh, vh, doh = one(q), one(k), one(v), one(do)
    lv = leaves_t[bb, :, h].cpu().numpy().astype(np.int64)  # (L, S)
    NL = L // LB
    T = round(math.log(NL, b))
    C = O.summaries(kh[None, :, None], b, LB, mode)  # (1, 1, NS, D)
    s_, t_, j_ = np.meshgrid(np.arange(S), np.arange(T), np.arange(b), indexing="ij")
    flat = ((((bb * L + np.arange(L)[:, None, None, None]) * H + h) * S + s_[None]) * T + t_[None]) * b + j_[None]
    U = uniforms_at(0, flat.reshape(-1)).reshape(1, L, 1, S, T, b)
    idx_o, _, margins = O.tree_sample(qh[None, :, None], C, b, LB, U, causal, N=L)
    clean = margins.min(axis=-1)[0, :, 0] > 1e-3
    assert not ((lv != idx_o[0, :, 0]) & clean).any(), f"{int(((lv != idx_o[0, :, 0]) & clean).sum())} clean differ"
    assert clean.mean() > 0.9
    print(f"  clean {clean.mean():.4f}, near-tie flips {int((lv != idx_o[0, :, 0]).sum())}", flush=True)
    r = O.head_fwd_bwd(qh, kh, vh, doh, C[0, 0], b, LB, lv, causal, 1.0 / math.sqrt(D))
    dk_ref = r["dk_leaf"] + O.pool_adjoint(r["dC"][None, None], L, b, LB, mode)[0, :, 0]
    assert rel(w[bb, :, h].cpu().numpy(), r["weights"]) < 1e-4
    for nm, got, ref in (("out", out, r["out"]), ("dq", dq, r["dq"]), ("dk", dk, dk_ref), ("dv", dv, r["dv"])):
        e = rel(one(got), ref)
        print(f"  {nm} rel err {e:.3g}", flush=True)
        assert e < 2e-2, (nm, e)


# The reference's own tree (binary, one token per leaf, Haar keys) at L=16384:
# the sampler evaluates its deep levels per sampled path and the backward runs
# them in node-major bands, so memory and work stay linear in L.
REF = (2, 16384, 16, 128, torch.bfloat16, 16)


@pytest.mark.parametrize("causal", [False, True])
def test_reference_tree_full_size(causal):
    """Non-causal: one complete (batch, head) against the oracle (leaves,
    weights, out, dq, dk, dv); causal (the reference's coupled sampler and
    hybrid head): the last 64 queries' leaves, out and dq rows against the
    float64 restatement on the GPU's own paths.  Both: the workspace is linear
    in L and the whole-problem identities hold."""
    from oracle import ref_torch as R
    from treeattention_amd import _lib
    from treeattention_amd.function import TreeOptions, make_problem, record_views, tree_backward, tree_forward

    B, L, H, D, dtype, S = REF
    print(f"[case] reference tree full size causal={causal}: B={B} L={L} H={H} D={D} S={S}", flush=True)
    q, k, v, do = inputs(B, L, H, D, dtype, "normal")
    opts = TreeOptions(num_samples=S, branching=2, leaf_block=1, tree_mode="compat", causal=causal, seed=0)
    _, fws, bws = _lib.byte_sizes(make_problem(q, k, v, opts))
    per_qh = (fws + bws) / (B * L * H)
    print(f"  workspaces {fws / 2**30:.2f} + {bws / 2**30:.2f} GiB ({per_qh / 1024:.1f} KiB per query-head)", flush=True)
    assert per_qh < 16 * 1024  # linear in L: a few KiB per query-head (the dense G^T would be 64 KiB)
    out, w, rec = tree_forward(q, k, v, opts)
    leaves_t, _ = record_views(q, k, v, opts, rec)
    dq, dk, dv = tree_backward(q, k, v, w, rec, do, opts)
    torch.cuda.synchronize()
    for t in (out, dq, dk, dv):
        assert torch.isfinite(t.float()).all()
    assert (w >= 0).all() and (w.sum(-1) - 1).abs().max().item() < 1e-5
    assert rel(dv.float().sum(1).cpu().numpy(), do.float().sum(1).cpu().numpy()) < 2e-2
    dkf = dk.float()
    assert (dkf.sum(1).norm(dim=-1) / dkf.pow(2).sum((1, 3)).sqrt()).max().item() < 2e-2
    T = 14
    bb, h = B - 1, H - 1
    one = lambda t: t[bb, :, h].float().cpu().numpy().astype(np.float64)  # noqa: E731  (L, D)
    qh, kh, vh, doh = one(q), one(k), one(v), one(do)
    lv = leaves_t[bb, :, h].cpu().numpy().astype(np.int64)  # (L, S)
    if not causal:
        C = O.summaries(kh[None, :, None], 2, 1, "compat")
        s_, t_, j_ = np.meshgrid(np.arange(S), np.arange(T), np.arange(2), indexing="ij")
        flat = ((((bb * L + np.arange(L)[:, None, None, None]) * H + h) * S + s_[None]) * T + t_[None]) * 2 + j_[None]
        U = uniforms_at(0, flat.reshape(-1)).reshape(1, L, 1, S, T, 2)
        idx_o, _, margins = O.tree_sample(qh[None, :, None], C, 2, 1, U, False, N=L)
        clean = margins.min(axis=-1)[0, :, 0] > 1e-3
        assert not ((lv != idx_o[0, :, 0]) & clean).any()
        assert clean.mean() > 0.9
        r = O.head_fwd_bwd(qh, kh, vh, doh, C[0, 0], 2, 1, lv, False, 1.0 / math.sqrt(D))
        dk_ref = r["dk_leaf"] + O.pool_adjoint(r["dC"][None, None], L, 2, 1, "compat")[0, :, 0]
        assert rel(w[bb, :, h].cpu().numpy(), r["weights"]) < 1e-4
        for nm, got, ref in (("out", out, r["out"]), ("dq", dq, r["dq"]), ("dk", dk, dk_ref), ("dv", dv, r["dv"])):
            e = rel(one(got), ref)
            print(f"  {nm} rel err {e:.3g}", flush=True)
            assert e < 2e-2, (nm, e)
        return
    # causal: the last SUB query positions, every (batch, head) of them -- the
    # reference's sampler couples all (batch, head, sample) lanes of a position
    t0 = L - SUB
    allq = lambda t: t.float().cpu().numpy().astype(np.float64).transpose(1, 0, 2, 3)  # noqa: E731  (L, B, H, D)
    qa, ka, va, da_ = allq(q), allq(k), allq(v), allq(do)
    kn = torch.tensor(O.haar_inorder(ka))  # (L-1, B, H, D) heap-ordered node keys
    bb_, ll_, hh_, s_, t_, j_ = np.meshgrid(np.arange(B), np.arange(t0, L), np.arange(H), np.arange(S), np.arange(T),
                                            np.arange(2), indexing="ij")
    flat = (((((bb_ * L + ll_) * H + hh_) * S + s_) * T + t_) * 2 + j_).reshape(-1)
    U = np.full((B, L, H, S, T, 2), 0.5, dtype=np.float32)
    U[:, t0:] = uniforms_at(0, flat).reshape(B, SUB, H, S, T, 2)
    qs = torch.tensor(qa[t0:], requires_grad=True)
    idx_o, _, margins, _ = R.sample_causal(qs.detach(), kn, L, U, offset=t0)
    clean = margins.numpy().min(axis=-1) > 1e-3
    lvs = leaves_t[:, t0:].cpu().numpy().astype(np.int64).transpose(1, 0, 2, 3)  # (SUB, B, H, S)
    assert not ((lvs != idx_o.numpy()) & clean).any(), f"{int(((lvs != idx_o.numpy()) & clean).sum())} clean differ"
    assert clean.mean() > 0.9
    idx, lp, _, _ = R.sample_causal(qs, kn, L, U, offset=t0, forced=torch.tensor(lvs))
    wr = torch.softmax(lp, dim=-1)  # (SUB, B, H, S)
    vb = torch.tensor(va).permute(1, 2, 0, 3)  # (B, H, L, D)
    gi = idx.clamp(0, L - 1).permute(1, 2, 0, 3).reshape(B, H, -1, 1).expand(-1, -1, -1, D)
    vg = torch.gather(vb, 2, gi).reshape(B, H, SUB, S, D).permute(2, 0, 1, 3, 4)
    o_ref = (wr[..., None] * vg).sum(-2)  # (SUB, B, H, D)
    o_ref.backward(torch.tensor(da_[t0:]))
    assert rel(w[:, t0:].cpu().numpy().transpose(1, 0, 2, 3), wr.detach().numpy()) < 1e-4
    for nm, got, ref in (("out", allq(out)[t0:], o_ref.detach().numpy()), ("dq", allq(dq)[t0:], qs.grad.numpy())):
        e = rel(got, ref)
        print(f"  {nm} rel err {e:.3g} (last {SUB} positions, all heads)", flush=True)
        assert e < 2e-2, (nm, e)
