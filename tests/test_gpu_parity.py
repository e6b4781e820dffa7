"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs.

Bar (from the task's north star):
* sampled leaf blocks bit-exact for every sample whose decisions all have a
  perturbed-score margin above 1e-3 (margins from the float64 oracle);
* outputs and gradients within 1e-5 (float32) / 2e-2 (bf16, fp16) norm-wise
  relative error, with the oracle evaluated on the GPU's sampled paths so a
  near-tie flip cannot hide or fake a numerics error.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import tree_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def rel(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make_inputs(B, L, H, D, dtype, seed=0, kind="normal", N=None):
    """q, k, v, dout as CPU tensors of ``dtype`` (torch.Generator, order q, k, v, dout)."""
    N = L if N is None else N
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, H, D, generator=g)
    k = torch.randn(B, N, H, D, generator=g)
    v = torch.randn(B, N, H, D, generator=g)
    do = torch.randn(B, L, H, D, generator=g)
    if kind == "scaled":
        q, k, v = (x / math.sqrt(D) for x in (q, k, v))
    elif kind == "skewed":  # Student-t(3) keys, queries with a shared direction x3
        z = torch.randn(B, N, H, D, generator=g)
        chi = (torch.randn(3, B, N, H, 1, generator=g) ** 2).sum(0) / 3
        k = z / chi.sqrt()
        u = torch.randn(D, generator=g)
        q = q + 3 * u / u.norm()
    return [x.to(dtype) for x in (q, k, v, do)]


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def run_case(B, L, H, D, S, b, LB, mode, causal, dtype, seed=0, kind="normal", backward=True, scale=None, N=None,
             dense_cols=0):
    from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

    N = L if N is None else N
    print(f"[case] B={B} L={L} N={N} H={H} D={D} S={S} b={b} LB={LB} mode={mode} causal={causal} {dtype} {kind} "
          f"dense_cols={dense_cols}", flush=True)
    q, k, v, do = make_inputs(B, L, H, D, dtype, seed, kind, N=N)
    nl = N // LB
    T = O.tree_depth(nl, b)
    U = O.uniforms(seed, (B, L, H, S, T, b))
    dev = torch.device("cuda:0")
    qg, kg, vg, dog = (x.to(dev) for x in (q, k, v, do))
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode=mode, causal=causal, scale=scale, seed=seed,
                       dense_cols=dense_cols)
    out, w, rec = tree_forward(qg, kg, vg, opts, torch.from_numpy(U).to(dev))
    leaves_t, sums_t = record_views(qg, kg, vg, opts, rec)
    torch.cuda.synchronize()
    leaves = leaves_t.cpu().numpy().astype(np.int64)

    q64, k64, v64, do64 = f64(q), f64(k), f64(v), f64(do)
    C = O.summaries(k64, b, LB, mode)
    sc = scale if scale is not None else 1.0 / math.sqrt(D)

    # K1: summaries (device layout pads every level to a multiple of 32 rows)
    off = O.level_offsets(b, T)
    sums = sums_t.cpu().numpy().reshape(B, H, -1, D)
    pad = 0
    for lam in range(1, T + 1):
        n = b**lam
        np.testing.assert_allclose(sums[:, :, pad:pad + n], C[:, :, off[lam]:off[lam] + n], rtol=2e-5, atol=2e-6)
        pad += (n + 31) // 32 * 32

    # K2: paths against the oracle's own sampling
    idx_o, lp_o, margins = O.tree_sample(q64, C, b, LB, U, causal, N=N)
    clean = margins.min(axis=-1) > 1e-3
    mism = (leaves != idx_o)
    assert not (mism & clean).any(), f"{int((mism & clean).sum())} clean samples differ"
    assert clean.mean() > 0.9
    if causal:
        blk = ((np.arange(L) + N - L) // LB)[None, :, None, None]
        assert (leaves <= blk).all()

    # K2 weights + K3 output, oracle on the GPU's paths
    lp_ref = O.path_logprobs(q64, C, b, nl, leaves)
    w_ref = O.sample_weights(lp_ref)
    o_s, _ = O.leaf_attention(q64, k64, v64, leaves, LB, causal, sc)
    out_ref = np.einsum("blhs,blhsd->blhd", w_ref, o_s)
    tol = TOL[dtype]
    assert rel(w.cpu().numpy(), w_ref) < max(tol, 1e-5), rel(w.cpu().numpy(), w_ref)
    assert rel(f64(out), out_ref) < tol, rel(f64(out), out_ref)
    assert torch.isfinite(out.float()).all()

    if backward:
        dq, dk, dv = tree_backward(qg, kg, vg, w, rec, dog, opts)
        dq_o, dC, dk_leaf, dv_o = O.tree_backward(q64, k64, v64, C, b, LB, leaves, w_ref, do64, causal, sc)
        dk_o = dk_leaf + O.pool_adjoint(dC, N, b, LB, mode)
        for name, got, ref in (("dq", dq, dq_o), ("dk", dk, dk_o), ("dv", dv, dv_o)):
            r = rel(f64(got), ref)
            print(f"  {name} rel err {r:.3g}", flush=True)
            assert r < tol, (name, r)
    return out, w, rec


def test_uniforms_match_oracle_bitwise():
    from treeattention_amd import _lib

    lib = _lib.load()
    n = 100003
    out = torch.empty(n, device="cuda:0", dtype=torch.float32)
    _lib.check(lib.ta_fill_uniforms(12345, n, out.data_ptr(), torch.cuda.current_stream().cuda_stream))
    ref = O.uniforms(12345, (n,))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_tree_lb1(dtype):
    run_case(2, 64, 2, 32, 4, 2, 1, "compat", False, dtype)


def test_c1_reference_plumbing_full_size():
    # BASELINE C1: B=1 L=1024 H=4 D=64 fp32, b=2, LB=16, S=4, non-causal, seed 0
    run_case(1, 1024, 4, 64, 4, 2, 16, "compat", False, torch.float32)


@pytest.mark.parametrize("mode", ["compat", "natural"])
def test_c2_like_binary_lb64(mode):
    run_case(2, 1024, 2, 64, 8, 2, 64, mode, False, torch.bfloat16)


@pytest.mark.parametrize("causal", [True, False])
def test_c3_like_branching4(causal):
    run_case(1, 1024, 2, 128, 16, 4, 64, "natural", causal, torch.bfloat16)


def test_c4_like_lb128_scaled():
    run_case(1, 1024, 2, 128, 16, 2, 128, "compat", False, torch.bfloat16, kind="scaled")


@pytest.mark.parametrize("D", [32, 96])
def test_c5_like_skewed_fp16_causal(D):
    run_case(2, 512, 2, D, 8, 2, 32, "compat", True, torch.float16, kind="skewed")


def test_fp32_causal_natural_b4():
    run_case(1, 256, 2, 64, 8, 4, 16, "natural", True, torch.float32)


# Deep levels evaluated per sampled path (sampler) and in node-major bands
# (backward): dense_cols caps the levels that run as dense tiles, so small
# problems take the paths that wide trees (the reference tree at long L) take.
@pytest.mark.parametrize("dtype,S", [(torch.float32, 8), (torch.bfloat16, 16)])
def test_sparse_levels_reference_tree(dtype, S):
    run_case(2, 256, 2, 64, S, 2, 1, "compat", False, dtype, dense_cols=8)  # levels 3..7 sparse, one 5-depth band


def test_sparse_levels_two_bands_lb16():
    run_case(1, 2048, 2, 64, 8, 2, 16, "compat", False, torch.bfloat16, dense_cols=4)  # leaf dq rows + 2 bands


def test_sparse_levels_b4_causal():
    run_case(1, 1024, 2, 128, 16, 4, 4, "natural", True, torch.bfloat16, dense_cols=16)


@pytest.mark.parametrize("D", [32, 96])
def test_sparse_levels_natural_b2_skewed_fp16(D):
    run_case(2, 512, 2, D, 8, 2, 2, "natural", True, torch.float16, kind="skewed", dense_cols=16)


def test_sparse_levels_fp32_natural_b2_causal_N_gt_L():
    run_case(1, 200, 2, 64, 8, 2, 1, "natural", True, torch.float32, N=256, dense_cols=4)


@pytest.mark.parametrize("b,L,LB,causal", [(2, 8192, 16, False), (4, 4096, 4, True)])
def test_levels_wider_than_one_sampler_pass(b, L, LB, causal):
    # 512 / 1024 leaf blocks: the deepest levels take two / four passes of the
    # sampler's 256-column logit tile, so an item that moved in one pass must
    # not decide again in a later pass of the same level
    run_case(1, L, 1, 32, 4, b, LB, "natural", causal, torch.bfloat16)


@pytest.mark.parametrize("S,b,LB,L,D,causal,dtype", [(32, 4, 16, 1024, 64, True, torch.bfloat16),
                                                     (64, 2, 8, 512, 32, False, torch.float32),
                                                     (24, 2, 4, 1024, 128, True, torch.bfloat16),
                                                     (48, 4, 16, 1024, 64, False, torch.float16),
                                                     (20, 8, 8, 512, 32, True, torch.float32),
                                                     (40, 8, 1, 512, 32, False, torch.bfloat16)])
def test_more_than_sixteen_samples(S, b, LB, L, D, causal, dtype):
    # 8 (S <= 32) or 16 (query, sample) items per sampler thread and 32- or
    # 64-lane groups per query in the tree-gradient scans, branching 2 and 4
    # specialized, 8 generic
    run_case(1, L, 2, D, S, b, LB, "natural", causal, dtype)


@pytest.mark.parametrize("S", [24, 64])
def test_more_than_sixteen_samples_reference_tree(S):
    # the reference's default of 64 paths on its own tree, per-path levels forced on
    run_case(1, 1024, 2, 64, S, 2, 1, "compat", False, torch.bfloat16, dense_cols=64)


@pytest.mark.parametrize("b,LB,L,causal", [(8, 1, 512, False), (16, 16, 4096, True)])
def test_branching_eight_and_sixteen(b, LB, L, causal):
    # branching outside {2, 4}: the runtime-b sampler and tree-gradient paths
    run_case(1, L, 2, 64, 8, b, LB, "natural", causal, torch.bfloat16)


@pytest.mark.parametrize("b,LB,L,D,causal,dtype", [(2, 7, 112, 96, True, torch.bfloat16),
                                                   (4, 3, 192, 64, False, torch.bfloat16),
                                                   (2, 48, 384, 128, True, torch.float16)])
def test_odd_leaf_blocks_and_partial_query_tiles(b, LB, L, D, causal, dtype):
    # leaf blocks that are not a power of two (padded key tiles), L not a
    # multiple of the 64-query tile
    run_case(2, L, 2, D, 8, b, LB, "natural", causal, dtype)


@pytest.mark.parametrize("D,LB,causal", [(128, 64, True), (96, 128, False), (64, 128, True), (128, 128, True)])
def test_float_large_leaf_tiles(D, LB, causal):
    # fp32 with large head dims / blocks: the leaf backward's 32- and 16-pair tiles (D=128, LB=128:
    # V operands from global memory)
    run_case(1, 16 * LB, 2, D, 8, 2, LB, "natural", causal, torch.float32)


def test_large_bucket_histogram():
    # 2048 leaf blocks (one counting-sort window) x 64 query chunks: the bucket
    # counts are scanned in segments by several workgroups per (batch, head)
    run_case(1, 16384, 1, 32, 4, 2, 8, "natural", False, torch.bfloat16)


@pytest.mark.parametrize("B,H,L,b,LB,S,causal", [(1, 1, 16384, 4, 4, 4, False), (2, 2, 8192, 2, 2, 8, True),
                                                (2, 8, 4096, 2, 1, 4, False)])
def test_bucketing_by_radix_sort(B, H, L, b, LB, S, causal):
    # more than 2048 leaf blocks: pairs are bucketed by a stable radix sort of
    # (batch * head, leaf block) keys (two or three 8-bit passes here), whose order
    # must equal the counting sort's (query order within a block)
    run_case(B, L, H, 32, S, b, LB, "natural", causal, torch.bfloat16, dense_cols=64 if LB == 1 else 0)


@pytest.mark.parametrize("causal", [False, True])
def test_fewer_queries_than_keys(causal):
    # L = 256 queries over N = 1024 keys (causal: bottom-right aligned)
    run_case(1, 256, 2, 64, 8, 2, 16, "compat", causal, torch.bfloat16, N=1024)


def test_causal_level_wider_than_one_chunk():
    # 256 leaf blocks: the deepest level spans two 128-column chunks of the
    # tree-gradient kernel, and the second is out of causal reach for the
    # first half of the query tiles (its products are skipped)
    run_case(1, 4096, 1, 32, 4, 2, 16, "natural", True, torch.bfloat16)


def test_seed_path_equals_explicit_uniforms_and_is_deterministic():
    from treeattention_amd.function import TreeOptions, record_views, tree_backward, tree_forward

    B, L, H, D, S, b, LB = 1, 1024, 2, 128, 16, 4, 64
    q, k, v, do = (x.cuda() for x in make_inputs(B, L, H, D, torch.bfloat16, 3))
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode="natural", causal=True, seed=77)
    U = torch.from_numpy(O.uniforms(77, (B, L, H, S, 2, b))).cuda()
    o1, w1, r1 = tree_forward(q, k, v, opts)
    o2, w2, r2 = tree_forward(q, k, v, opts, U)
    o3, w3, r3 = tree_forward(q, k, v, opts)
    assert torch.equal(o1, o2) and torch.equal(w1, w2) and torch.equal(o1, o3) and torch.equal(w1, w3)
    # the record's meaningful content (sampled leaves, summaries) is reproducible;
    # its unused slots are scratch and are not compared
    for a, c in zip(record_views(q, k, v, opts, r1), record_views(q, k, v, opts, r3)):
        assert torch.equal(a, c)
    g1 = tree_backward(q, k, v, w1, r1, do, opts)
    g2 = tree_backward(q, k, v, w3, r3, do, opts)
    for a, c in zip(g1, g2):
        assert torch.equal(a, c)


@pytest.mark.parametrize("view", ["head_slice", "fused_qkv"])
def test_strided_views_with_gaps(view):
    """q / k / v as views with gaps between rows (a slice of the heads, or q, k, v inside one
    fused (B, L, 3, H, D) tensor): the same results, bit for bit, as contiguous copies, with the
    gradients in buffers of the views' shapes."""
    from treeattention_amd.function import TreeOptions, tree_backward, tree_forward

    B, L, H, D, S, b, LB = 1, 512, 4, 64, 8, 2, 16
    print(f"[case] strided views {view}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    if view == "head_slice":
        big = [torch.randn(B, L, 2 * H, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3)]
        q, k, v = (t[:, :, H:] for t in big)
    else:
        qkv = torch.randn(B, L, 3, H, D, device="cuda", generator=g).to(torch.bfloat16)
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    do = torch.randn(B, L, H, D, device="cuda", generator=g).to(torch.bfloat16)
    opts = TreeOptions(num_samples=S, branching=b, leaf_block=LB, tree_mode="natural", causal=True, seed=4)
    o1, w1, r1 = tree_forward(q, k, v, opts)
    grads1 = tree_backward(q, k, v, w1, r1, do, opts)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    o2, w2, r2 = tree_forward(qc, kc, vc, opts)
    grads2 = tree_backward(qc, kc, vc, w2, r2, do, opts)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(w1, w2)
    for a, c in zip(grads1, grads2):
        assert a.shape == c.shape and torch.equal(a, c)


# (L, B, H, D, S) of the reference's own end-to-end parity test
# (test_harness_smoke.py:824-917); D = 16 runs zero-padded to 32 head dims.
REFERENCE_E2E_SHAPES = [(8, 1, 2, 16, 4), (32, 2, 2, 16, 4), (64, 1, 8, 16, 4), (128, 1, 2, 64, 8), (512, 2, 4, 32, 8),
                        (32, 2, 2, 32, 4),
                        # head dims that are not a kernel size nor a multiple of 8 (E % H == 0 is all the
                        # reference asks, _tree_mha.py:348-351): zero-padded to 32 / 128
                        (64, 1, 2, 5, 4), (128, 2, 3, 100, 8)]


@pytest.mark.parametrize("L,B,H,D,S", REFERENCE_E2E_SHAPES)
def test_op_level_hierarchical_attention_matches_reference_restatement(L, B, H, D, S):
    """Reference op signature (L,B,E) with heap node keys, against ``ref_forward_non_causal``:
    sampled leaves equal wherever every decision's margin exceeds 1e-3; weights, output and
    gradients against the restatement on the GPU's own paths (returned packed, the reference's
    record format)."""
    import treeattention_amd as ta

    print(f"[case] op-level L={L} B={B} H={H} D={D} S={S}", flush=True)
    E = H * D
    g = torch.Generator().manual_seed(1234)
    query = torch.randn(L, B, E, generator=g)
    key = torch.randn(L - 1, B, E, generator=g)
    value = torch.randn(L, B, E, generator=g)
    gout = torch.randn(L, B, E, generator=g)
    T = int(math.log2(L))
    U = O.uniforms(0, (B, L, H, S, T, 2))
    qd, kd, vd = (x.cuda().requires_grad_(True) for x in (query, key, value))
    out, w, paths = ta.hierarchical_attention(qd, kd, vd, num_heads=H, num_samples=S,
                                              uniforms=torch.from_numpy(U).cuda(), return_paths=True)
    out.backward(gout.cuda())
    q4 = query.double().numpy().reshape(L, B, H, D)
    k4 = key.double().numpy().reshape(L - 1, B, H, D)
    v4 = value.double().numpy().reshape(L, B, H, D)
    qb, vb = q4.transpose(1, 0, 2, 3), v4.transpose(1, 0, 2, 3)
    C = O.nodekeys_to_summaries(k4.transpose(1, 2, 0, 3))
    # paths: the restatement's sampling, compared where no decision is within 1e-3
    gum = O.gumbel(U).transpose(1, 0, 2, 3, 4, 5)
    _, _, ref_idx = O.ref_forward_non_causal(q4, k4, v4, gum)
    _, _, margins = O.tree_sample(qb, C, 2, 1, U, False)
    leaves = O.unpack_paths(paths.cpu().numpy(), L).transpose(1, 0, 2, 3)  # (B, L, H, S)
    clean = margins.min(axis=-1) > 1e-3
    mism = leaves != ref_idx.transpose(1, 0, 2, 3)
    assert not (mism & clean).any(), f"{int((mism & clean).sum())} clean samples differ"
    assert clean.mean() > 0.9
    # weights and output on the GPU's paths
    wb = O.sample_weights(O.path_logprobs(qb, C, 2, L, leaves))
    o_s, _ = O.leaf_attention(qb, np.zeros_like(vb), vb, leaves, 1, False, 1.0)
    out_ref = np.einsum("blhs,blhsd->blhd", wb, o_s)
    assert rel(f64(out), out_ref.transpose(1, 0, 2, 3).reshape(L, B, E)) < 1e-5
    assert rel(w.detach().cpu().numpy(), wb.transpose(1, 0, 2, 3)) < 1e-5
    # gradients: explicit oracle backward on the node-key tree
    dq, dC, _, dv = O.tree_backward(qb, np.zeros_like(vb), vb, C, 2, 1, leaves, wb,
                                    gout.double().numpy().reshape(L, B, H, D).transpose(1, 0, 2, 3), False)
    dkn = O.nodekeys_adjoint(dC)  # (B,H,K,D)
    assert rel(f64(qd.grad).reshape(L, B, H, D).transpose(1, 0, 2, 3), dq) < 1e-5
    assert rel(f64(kd.grad).reshape(L - 1, B, H, D).transpose(1, 2, 0, 3), dkn) < 1e-5
    assert rel(f64(vd.grad).reshape(L, B, H, D).transpose(1, 0, 2, 3), dv) < 1e-5


@pytest.mark.parametrize("D,dtype", [(40, torch.bfloat16), (12, torch.float32)])
def test_head_dim_padding_is_exact(D, dtype):
    """A head dim the kernels do not implement runs zero-padded to the next one with the softmax
    scale of the true D: output and gradients equal the padded problem's, sliced."""
    import treeattention_amd as ta

    B, L, H, S = 1, 512, 2, 8
    Dp = 64 if D > 32 else 32
    print(f"[case] head-dim padding D={D} -> {Dp} {dtype}", flush=True)
    g = torch.Generator().manual_seed(5)
    q, k, v, do = (torch.randn(B, L, H, D, generator=g).to(dtype).cuda() for _ in range(4))
    kw = dict(num_samples=S, branching=2, leaf_block=16, tree_mode="natural", seed=11)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v)]
    out = ta.tree_attention(*xs, True, None, **kw)
    out.backward(do)
    pad = lambda t: torch.nn.functional.pad(t, (0, Dp - D))  # noqa: E731
    ps = [pad(x).requires_grad_(True) for x in (q, k, v)]
    outp = ta.tree_attention(*ps, True, 1.0 / math.sqrt(D), **kw)
    outp.backward(pad(do))
    assert out.shape == (B, L, H, D)
    assert torch.equal(out, outp[..., :D])
    for a_, b_ in zip(xs, ps):
        assert torch.equal(a_.grad, b_.grad[..., :D])


def test_op_level_block_size_invariance():
    """The reference streams its sampler over query blocks of ``block_size``; the result does not
    depend on it (its own block-size test, test_harness_smoke.py:391-421)."""
    import treeattention_amd as ta

    L, B, H, D, S = 64, 1, 2, 32, 4
    g = torch.Generator().manual_seed(7)
    query, key, value = (torch.randn(n, B, H * D, generator=g).cuda() for n in (L, L - 1, L))
    outs = [ta.hierarchical_attention(query, key, value, num_heads=H, num_samples=S, block_size=bs, seed=3)
            for bs in (1, 7, 64, 256)]
    for o, w in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(w, outs[0][1])


def test_op_level_edge_cases():
    import treeattention_amd as ta

    L, B, H, D = 8, 1, 2, 32
    q = torch.randn(L, B, H * D, device="cuda")
    v1 = torch.randn(1, B, H * D, device="cuda")
    out, w = ta.hierarchical_attention(q, v1[:0], v1, num_heads=H, num_samples=4)
    assert torch.equal(out, v1.expand(L, -1, -1)) and w.shape == (L, B, H, 1)
    with pytest.raises(ValueError):
        ta.hierarchical_attention(q, torch.randn(3, B, H * D, device="cuda"), torch.randn(8, B, H * D, device="cuda"),
                                  num_heads=H, num_samples=4)


def test_attn_fn_adapter_contract(monkeypatch):
    import treeattention_amd as ta

    monkeypatch.setenv("TREEATTN_NUM_SAMPLES", "8")
    monkeypatch.setenv("TREEATTN_BRANCHING", "4")
    monkeypatch.setenv("TREEATTN_LEAF_BLOCK", "64")
    monkeypatch.setenv("TREEATTN_TREE_MODE", "natural")
    ad = ta.adapter()
    B, L, H, D = 2, 1024, 4, 64
    q, k, v, do = (x.cuda() for x in make_inputs(B, L, H, D, torch.bfloat16, 5))
    for t in (q, k, v):
        t.requires_grad_(True)
    ptrs = [t.data_ptr() for t in (q, k, v)]
    snap = [t.detach().clone() for t in (q, k, v)]
    out = ad.fn(q, k, v, True, None)
    out2 = ad.fn(q, k, v, True, None)
    assert out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous()
    assert torch.equal(out, out2)  # deterministic forward
    out.backward(do)
    assert [t.data_ptr() for t in (q, k, v)] == ptrs
    for t, s in zip((q, k, v), snap):
        assert torch.equal(t.detach(), s)  # inputs untouched
    assert all(torch.isfinite(t.grad.float()).all() for t in (q, k, v))
