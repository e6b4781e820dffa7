"""Autograd Functions over the HIP library.

``DeterministicTreeAttention`` / ``DeterministicAdapterAttention`` run the
reference's exact mode (``_tree_mha.py:271-321``); see the section below.

``TreeAttentionFunction`` is the MI355X counterpart of treeattn-cuda's
``_StochasticNonCausalTreeAttention`` (``_autograd.py:645-860``): the forward
samples paths and combines the leaf outputs, saves a compact record (the
sampled leaf blocks, their weights and the per-leaf-block bucket), and the
backward replays nothing on the host: one call produces dq, dk, dv.  The
sample weights are returned as a non-differentiable output, as in the
reference (``_autograd.py:703``).
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
from dataclasses import dataclass

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.TA_F32, torch.bfloat16: _lib.TA_BF16, torch.float16: _lib.TA_F16}


@dataclass(frozen=True)
class TreeOptions:
    """How the tree is built and sampled.

    * ``num_samples``: paths per query (1..1024; above 64 in chunks of at most 64,
      non-causal or exact causal).
    * ``branching``, ``leaf_block``: ``N = leaf_block * branching**T``.
    * ``tree_mode``: ``"compat"`` (reference key layout: in-order Haar of the
      leaf-block means, read in heap order), ``"natural"`` (child summary =
      half the mean key of the child's subtree) or ``"nodekeys"`` (``k`` holds
      the heap-ordered node keys, the op-level reference API).
    * ``causal``: causal attention, with ``causal_mode``:

      - ``"reference"``: the reference's causal stochastic mode
        (``_tree_mha.py:125-268,379-394``), for the reference tree only
        (``branching=2, leaf_block=1``, compat or node-key summaries): query
        ``t`` has boundary leaf ``t``; decisions are corrected by the boundary
        log-masses while every (batch, head, sample) lane of the query is on
        the boundary path, plain afterwards; with ``L > num_samples`` the first
        ``num_samples`` queries get exact causal attention;
      - ``"exact"``: bottom-right aligned mask with sampling restricted exactly
        to the allowed leaf blocks (any tree);
      - ``"auto"`` (default): ``"reference"`` on the reference tree, else
        ``"exact"``.
    * ``scale``: leaf-block softmax scale (``None`` -> ``1/sqrt(D)``).
    * ``max_logit``: child logits are clamped to ``+-max_logit/2``.
    * ``seed``: counter-RNG key for the Gumbel uniforms when no explicit
      ``uniforms`` tensor is given.
    * ``layout``: ``"bshd"`` (B, L, H, D) or ``"lbhd"`` (L, B, H, D).
    * ``dense_cols``: tree levels with at most this many children are
      evaluated as dense level tiles, wider ones per sampled path (0: the
      library's defaults, under which 16-bit inputs with b = 2 or 4,
      ``leaf_block >= 2`` and ``T*b <= 32`` take the backward's tree part
      along the sampled paths inside the leaf backward, and 16-bit one-token
      binary leaves outside the reference causal mode per subtree of 64
      leaves); for tuning and tests, results change only by rounding.
    """

    num_samples: int
    branching: int = 2
    leaf_block: int = 1
    tree_mode: str = "compat"
    causal: bool = False
    causal_mode: str = "auto"
    scale: float | None = None
    max_logit: float = 1e3
    seed: int = 0
    layout: str = "bshd"
    dense_cols: int = 0


def _bl(t: torch.Tensor, layout: str) -> tuple[int, int]:
    """(batch, position) sizes of a 4-D tensor in ``layout``."""
    return (t.shape[0], t.shape[1]) if layout == "bshd" else (t.shape[1], t.shape[0])


def _strides(t: torch.Tensor, layout: str):
    s = t.stride()
    return (s[0], s[1], s[2]) if layout == "bshd" else (s[1], s[0], s[2])


def _prep(t: torch.Tensor) -> torch.Tensor:
    """Last dim contiguous, other strides multiples of 8, 16-byte aligned."""
    if t.stride(-1) != 1 or any(st % 8 for st in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _dense(t: torch.Tensor) -> torch.Tensor:
    """``t`` if its elements fill its span without gaps (any dim order), else a contiguous
    copy.  The backward writes dq / dk / dv with the strides of q / k / v into buffers from
    ``torch.empty_like``, which keeps the strides of dense tensors only: a view with gaps
    (a slice of heads, one of q / k / v inside a fused qkv tensor) would send the writes past
    the gradient's end."""
    expect = 1
    for st, n in sorted((st, n) for st, n in zip(t.stride(), t.shape) if n > 1):
        if st != expect:
            return t.contiguous()
        expect *= n
    return t


_HEAD_DIMS = (32, 64, 96, 128)


def _pad_heads(q, k, v, opts: TreeOptions):
    """Zero-pads the head dim to the next size the kernels implement (dots and
    value rows are unchanged by zero columns); the softmax scale keeps the true D."""
    D = q.shape[-1]
    if D > 128:
        raise NotImplementedError(f"the stochastic kernels take head dims up to 128 (got {D})")
    Dp = next(x for x in _HEAD_DIMS if x >= D)
    pad = lambda t: torch.nn.functional.pad(t, (0, Dp - D))  # noqa: E731
    scale = opts.scale if opts.scale is not None else 1.0 / math.sqrt(D)
    return pad(q), pad(k), pad(v), dataclasses.replace(opts, scale=scale)


def make_problem(q, k, v, opts: TreeOptions) -> _lib.Problem:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v must share one of {list(_DTYPES)} (got {q.dtype}, {k.dtype}, {v.dtype})")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("q, k, v must be on a GPU device")
    B, L = _bl(q, opts.layout)
    Bv, N = _bl(v, opts.layout)
    H, D = q.shape[2], q.shape[3]
    if Bv != B or v.shape[2] != H or v.shape[3] != D or k.shape[2] != H or k.shape[3] != D:
        raise ValueError(f"incompatible shapes q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if opts.tree_mode == "nodekeys":
        if _bl(k, opts.layout)[1] != N - 1:
            raise ValueError(f"Key tensor length must be N-1 ({N - 1}), but got {_bl(k, opts.layout)[1]}.")
    elif _bl(k, opts.layout)[1] != N:
        raise ValueError(f"k and v must have the same length (got {_bl(k, opts.layout)[1]} and {N})")
    p = _lib.Problem()
    p.B, p.L, p.H, p.D, p.N = B, L, H, D, N
    p.num_samples = opts.num_samples
    p.branching = opts.branching
    p.leaf_block = opts.leaf_block
    p.tree_mode = _lib.TREE_MODES[opts.tree_mode]
    p.causal = _causal_code(opts)
    p.dtype = _DTYPES[q.dtype]
    p.scale = float(opts.scale) if opts.scale is not None else 1.0 / math.sqrt(D)
    p.max_logit = float(opts.max_logit)
    p.dense_cols = int(opts.dense_cols)
    p.q_strides[:] = _strides(q, opts.layout)
    p.k_strides[:] = _strides(k, opts.layout)
    p.v_strides[:] = _strides(v, opts.layout)
    p.o_strides[:] = _strides(q, opts.layout)
    p.g_strides[:] = _strides(q, opts.layout)
    return p


def reference_tree(opts: TreeOptions) -> bool:
    """True for the reference's tree: binary, one token per leaf, Haar / node keys."""
    return opts.branching == 2 and opts.leaf_block == 1 and opts.tree_mode in ("compat", "nodekeys")


def _causal_code(opts: TreeOptions) -> int:
    if not opts.causal:
        return _lib.TA_CAUSAL_NONE
    mode = opts.causal_mode
    if mode == "auto":
        mode = "reference" if reference_tree(opts) else "exact"
    if mode not in ("reference", "exact"):
        raise ValueError(f"causal_mode must be 'auto', 'reference' or 'exact' (got {opts.causal_mode!r})")
    return _lib.TA_CAUSAL_REFERENCE if mode == "reference" else _lib.TA_CAUSAL_EXACT


def _weights_like(q: torch.Tensor, S: int, layout: str) -> tuple[torch.Tensor, tuple[int, int, int]]:
    w = torch.empty((*q.shape[:3], S), device=q.device, dtype=torch.float32)
    return w, _strides(w, layout)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def tree_forward(q, k, v, opts: TreeOptions, uniforms: torch.Tensor | None = None,
                 paths: torch.Tensor | None = None):
    """Forward only: returns ``(out, weights, record)``.  With ``paths``
    (packed path bits, ``(L, B, H, S, path_bytes)`` uint8, see
    ``pack_paths``) the given paths are replayed instead of sampled."""
    lib = _lib.load()
    D = q.shape[-1]
    if D not in _HEAD_DIMS:
        q, k, v, opts = _pad_heads(q, k, v, opts)
        out, weights, record = tree_forward(q, k, v, opts, uniforms, paths)
        return out[..., :D], weights, record
    q, k, v = _prep(q), _prep(k), _prep(v)
    prob = make_problem(q, k, v, opts)
    rec_b, fws_b, _ = _lib.byte_sizes(prob)
    out = torch.empty_like(q)
    prob.o_strides[:] = _strides(out, opts.layout)
    weights, ws = _weights_like(q, opts.num_samples, opts.layout)
    prob.w_strides[:] = ws
    record = torch.empty(rec_b, device=q.device, dtype=torch.uint8)
    work = torch.empty(fws_b, device=q.device, dtype=torch.uint8)
    if uniforms is not None:
        expect = (prob.B, prob.L, prob.H, opts.num_samples)
        if (uniforms.dtype != torch.float32 or not uniforms.is_contiguous() or uniforms.device != q.device
                or tuple(uniforms.shape[:4]) != expect or uniforms.dim() != 6
                or uniforms.shape[5] != opts.branching):
            raise ValueError(
                f"uniforms must be a contiguous float32 (B, L, H, S, T, b) tensor on {q.device}, "
                f"leading dims {expect}; got {tuple(uniforms.shape)} {uniforms.dtype}")
    if paths is not None:
        if uniforms is not None:
            raise ValueError("give either uniforms or paths, not both")
        if prob.causal != _lib.TA_CAUSAL_NONE:
            raise ValueError("path replay is for non-causal attention (as the reference's replay)")
        nl = prob.N // prob.leaf_block
        expect = (prob.L, prob.B, prob.H, opts.num_samples, path_bytes(nl))
        if (paths.dtype != torch.uint8 or not paths.is_contiguous() or paths.device != q.device
                or tuple(paths.shape) != expect):
            raise ValueError(f"paths must be a contiguous uint8 {expect} tensor on {q.device}; "
                             f"got {tuple(paths.shape)} {paths.dtype}")
    with torch.cuda.device(q.device):
        if paths is not None:
            _lib.check(lib.ta_forward_replay(ctypes.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             paths.data_ptr(), out.data_ptr(), weights.data_ptr(),
                                             record.data_ptr(), work.data_ptr(), _stream(q.device)))
        else:
            _lib.check(lib.ta_forward(ctypes.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(uniforms),
                                      ctypes.c_uint64(opts.seed & 0xFFFFFFFFFFFFFFFF), out.data_ptr(),
                                      weights.data_ptr(), record.data_ptr(), work.data_ptr(), _stream(q.device)))
    return out, weights, record


def tree_backward(q, k, v, weights, record, grad_out, opts: TreeOptions):
    """Backward from a forward record: returns ``(dq, dk, dv)``."""
    lib = _lib.load()
    D = q.shape[-1]
    if D not in _HEAD_DIMS:
        q, k, v, opts = _pad_heads(q, k, v, opts)
        grad_out = torch.nn.functional.pad(grad_out, (0, q.shape[-1] - D))
        dq, dk, dv = tree_backward(q, k, v, weights, record, grad_out, opts)
        return dq[..., :D], dk[..., :D], dv[..., :D]
    q, k, v = _dense(_prep(q)), _dense(_prep(k)), _dense(_prep(v))
    grad_out = _prep(grad_out)
    prob = make_problem(q, k, v, opts)
    prob.g_strides[:] = _strides(grad_out, opts.layout)
    prob.w_strides[:] = _strides(weights, opts.layout)
    _, _, bws_b = _lib.byte_sizes(prob)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    work = torch.empty(bws_b, device=q.device, dtype=torch.uint8)
    with torch.cuda.device(q.device):
        _lib.check(lib.ta_backward(ctypes.byref(prob), q.data_ptr(), k.data_ptr(), v.data_ptr(), grad_out.data_ptr(),
                                   weights.data_ptr(), record.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                   dv.data_ptr(), work.data_ptr(), _stream(q.device)))
    return dq, dk, dv


class TreeAttentionFunction(torch.autograd.Function):
    """``apply(q, k, v, opts, uniforms=None, paths=None) -> (out, weights)``."""

    @staticmethod
    def forward(ctx, q, k, v, opts: TreeOptions, uniforms=None, paths=None):
        out, weights, record = tree_forward(q, k, v, opts, uniforms, paths)
        ctx.save_for_backward(q, k, v, weights, record)
        ctx.opts = opts
        ctx.mark_non_differentiable(weights)
        return out, weights

    @staticmethod
    def backward(ctx, grad_out, grad_weights):
        del grad_weights
        q, k, v, weights, record = ctx.saved_tensors
        dq, dk, dv = tree_backward(q, k, v, weights, record, grad_out, ctx.opts)
        return dq, dk, dv, None, None, None


class StochasticTreeAttention(torch.autograd.Function):
    """Drop-in for treeattn-cuda's ``_StochasticNonCausalTreeAttention``.

    ``apply(q (L,B,H,D), k (N-1,B,H,D) heap-ordered node keys, v (N,B,H,D),
    num_samples, block_size, max_logit, is_causal=False, seed=0,
    uniforms=None, paths=None, return_paths=False) -> (out (L,B,H,D),
    weights (L,B,H,S) float32)``, gradients ``(dq, dk, dv, None, ...)``
    (``_autograd.py:645-707,860``).  ``block_size`` (the reference's query
    streaming) does not change results and is accepted for compatibility.
    Edge cases follow ``_autograd.py:660-683``.  ``paths``: packed path bits
    ``(L, B, H, S, ceil(log2(N)/8))`` uint8 (the reference's saved path
    record, ``_autograd.py:68-90``) to replay instead of sampling
    (non-causal); ``return_paths=True`` adds the forward's own packed paths
    as a third output.
    """

    @staticmethod
    def forward(ctx, q, k, v, num_samples, block_size=256, max_logit=1e3, is_causal=False, seed=0, uniforms=None,
                paths=None, return_paths=False):
        del block_size
        num_leaves = v.shape[0]
        if num_samples <= 0:
            raise ValueError(f"num_samples must be > 0, got {num_samples}")
        ctx.num_leaves = num_leaves
        if num_leaves <= 1:
            if num_leaves == 0:
                out = torch.zeros_like(q)
                weights = torch.empty((*q.shape[:-1], 0), device=q.device, dtype=q.dtype)
            else:
                out = v.expand(q.shape[0], -1, -1, -1).contiguous()
                weights = torch.ones((*q.shape[:-1], 1), device=q.device, dtype=q.dtype)
            ctx.save_for_backward(q, k, v)
            ctx.mark_non_differentiable(weights)
            if not return_paths:
                return out, weights
            packed = torch.zeros((*q.shape[:-1], int(num_samples), 0), device=q.device, dtype=torch.uint8)
            ctx.mark_non_differentiable(packed)
            return out, weights, packed
        if paths is not None and is_causal:
            raise ValueError("path replay is for non-causal attention (as the reference's replay)")
        opts = TreeOptions(num_samples=int(num_samples), branching=2, leaf_block=1, tree_mode="nodekeys",
                           causal=bool(is_causal), max_logit=float(max_logit), seed=int(seed), layout="lbhd")
        out, weights, record = tree_forward(q, k, v, opts, uniforms, paths)
        ctx.save_for_backward(q, k, v, weights, record)
        ctx.opts = opts
        packed = None
        if return_paths:
            leaves, _ = record_views(q, k, v, opts, record)
            packed = pack_paths(leaves, num_leaves, layout="blhs")
        if is_causal and q.shape[0] > num_samples:
            # hybrid: the first num_samples queries are exact; the reference returns the
            # sample weights of the other rows only (_tree_mha.py:379-413)
            weights = weights[num_samples:]
        ctx.mark_non_differentiable(weights)
        if packed is None:
            return out, weights
        ctx.mark_non_differentiable(packed)
        return out, weights, packed

    @staticmethod
    def backward(ctx, grad_out, grad_weights, *grad_paths):
        del grad_weights, grad_paths
        nones = (None,) * 8
        if ctx.num_leaves <= 1:
            q, k, v = ctx.saved_tensors
            dv = torch.zeros_like(v)
            if ctx.num_leaves == 1:
                dv[0] = grad_out.float().sum(dim=0).to(v.dtype)
            return (torch.zeros_like(q), torch.zeros_like(k), dv) + nones
        q, k, v, weights, record = ctx.saved_tensors
        dq, dk, dv = tree_backward(q, k, v, weights, record, grad_out, ctx.opts)
        return (dq, dk, dv) + nones


# ---------------------------------------------------------------------------
# Deterministic (exact) mode on the reference tree (_tree_mha.py:271-321).
# The node logits X = Q K^T and the products out = W V, dW = dout V^T,
# dq = G K, dK = G^T Q, dv = W^T dout are plain batched GEMMs (the BLAS
# library behind torch.matmul); the tree recursion over every row (weights,
# and the node-logit gradient G) runs in the library's HIP kernels.  Memory is
# that of the reference's mode: the (L, B, H, N) weights it returns, plus the
# logits.


def _bh(t: torch.Tensor) -> torch.Tensor:
    """(L, B, H, D) -> contiguous float32 (B, H, L, D)."""
    return t.permute(1, 2, 0, 3).float().contiguous()


def _on_device(*ts) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("tree attention runs on HIP device tensors; got a tensor on " + str(t.device))


def det_weights(q, k, N: int, causal: bool):
    """Exact leaf weights ``W (B,H,L,N)`` float32 of ``q (L,B,H,D)`` and node keys ``k (N-1,B,H,D)``."""
    _on_device(q, k)
    lib = _lib.load()
    L, B, H, _ = q.shape
    qf, kf = _bh(q), _bh(k)
    X = torch.matmul(qf, kf.transpose(-1, -2).contiguous())  # (B, H, L, N-1)
    W = torch.empty((B, H, L, N), device=q.device, dtype=torch.float32)
    with torch.cuda.device(q.device):
        _lib.check(lib.ta_det_weights(X.data_ptr(), N - 1, W.data_ptr(), N, B * H * L, L, N, int(bool(causal)),
                                      _stream(q.device)))
    return W


def det_forward(q, k, v, causal: bool):
    """``q (L,B,H,D)``, node keys ``k (N-1,B,H,D)``, ``v (N,B,H,D)`` -> ``(out (L,B,H,D)
    in v's dtype, W (B,H,L,N) float32)``."""
    _on_device(q, k, v)
    W = det_weights(q, k, v.shape[0], causal)
    out = torch.matmul(W.to(v.dtype), v.permute(1, 2, 0, 3).contiguous())  # weights cast to v's dtype (:318)
    return out.permute(2, 0, 1, 3), W


def det_stream_supported(q: torch.Tensor, N: int) -> bool:
    """Whether the streaming forward covers this case: 16-bit inputs, 64 <= N <= 32768, kernel head dim."""
    return q.dtype in (torch.bfloat16, torch.float16) and 64 <= N <= 32768 and q.shape[-1] in _HEAD_DIMS


def det_stream_forward(q, kn, v, causal: bool, layout: str = "bshd", return_lse: bool = False):
    """Exact tree attention without the ``(L, N)`` weights: ``q``, ``v`` in ``layout`` (``"bshd"`` or
    ``"lbhd"``), node keys ``kn (N-1, B, H, D)`` in q's dtype -> ``out`` (q's layout and dtype), and
    with ``return_lse`` the causal log-normalizer ``(B, H, L)`` float32 (None when not causal)."""
    _on_device(q, kn, v)
    lib = _lib.load()
    q, v, kn = _prep(q), _prep(v), _prep(kn.to(q.dtype))
    B, L = _bl(q, layout)
    H, D = q.shape[2], q.shape[3]
    N = v.shape[1] if layout == "bshd" else v.shape[0]
    out = torch.empty_like(q)
    lse = torch.empty((B, H, L), device=q.device, dtype=torch.float32) if causal else None
    qs, vs, os_ = ((ctypes.c_int64 * 3)(*_strides(t, layout)) for t in (q, v, out))
    ks = (ctypes.c_int64 * 3)(kn.stride(1), kn.stride(0), kn.stride(2))
    with torch.cuda.device(q.device):
        _lib.check(lib.ta_det_stream_forward(_DTYPES[q.dtype], q.data_ptr(), qs, kn.data_ptr(), ks, v.data_ptr(), vs,
                                             out.data_ptr(), os_, _ptr(lse), B, L, H, D, N, int(bool(causal)),
                                             _stream(q.device)))
    return (out, lse) if return_lse else out


def det_stream_backward(q, kn, v, grad_out, out, lse, causal: bool, layout: str = "bshd"):
    """Gradients of ``det_stream_forward``: ``(dq (q's layout and dtype), dkn (N-1, B, H, D) float32,
    dv (v's layout and dtype))``.  The 64-leaf subtrees' part runs in the library's streaming
    kernels; the ``N/64 - 1`` top nodes are the exact mode on a coarse tree whose leaves are the
    chunks (``ta_det_grad`` on the chunk totals, two small products)."""
    _on_device(q, kn, v, grad_out)
    lib = _lib.load()
    q, v, grad_out, kn = _prep(q), _prep(v), _prep(grad_out), _prep(kn.to(q.dtype))
    B, L = _bl(q, layout)
    H, D = q.shape[2], q.shape[3]
    N = v.shape[1] if layout == "bshd" else v.shape[0]
    NC = N // 64
    dev = q.device
    delta = None
    if causal:
        d = (grad_out.float() * out.float()).sum(-1)  # dout . out per row
        delta = (d.permute(0, 2, 1) if layout == "bshd" else d.permute(1, 2, 0)).contiguous()  # (B, H, L)
    dq_sub = torch.empty((B, H, L, D), device=dev, dtype=torch.float32)
    tot = torch.empty((B, H, L, NC), device=dev, dtype=torch.float32)
    dkn = torch.empty((N - 1, B, H, D), device=dev, dtype=torch.float32)
    dv = torch.empty_like(v)
    qs, gs, vs, dvs = ((ctypes.c_int64 * 3)(*_strides(t, layout)) for t in (q, grad_out, v, dv))
    ks = (ctypes.c_int64 * 3)(kn.stride(1), kn.stride(0), kn.stride(2))
    st = _stream(dev)
    with torch.cuda.device(dev):
        _lib.check(lib.ta_det_stream_backward(_DTYPES[q.dtype], q.data_ptr(), qs, grad_out.data_ptr(), gs,
                                              kn.data_ptr(), ks, v.data_ptr(), vs, _ptr(lse), _ptr(delta),
                                              dq_sub.data_ptr(), tot.data_ptr(), dkn.data_ptr(), dv.data_ptr(), dvs,
                                              B, L, H, D, N, int(bool(causal)), st))
        qf = (q.permute(0, 2, 1, 3) if layout == "bshd" else q.permute(1, 2, 0, 3)).float()  # (B, H, L, D)
        if NC >= 2:
            kt = kn[:NC - 1].float().permute(1, 2, 0, 3)  # (B, H, NC-1, D)
            X = torch.matmul(qf, kt.transpose(-1, -2).contiguous()).contiguous()  # top-node logits
            ones = torch.ones_like(tot)
            _lib.check(lib.ta_det_grad(X.data_ptr(), NC - 1, tot.data_ptr(), ones.data_ptr(), NC, B * H * L, NC, 0,
                                       st))
            dq_sub += torch.matmul(X, kt)
            dkn[:NC - 1] = torch.matmul(X.transpose(-1, -2), qf).permute(2, 0, 1, 3)
    dq = (dq_sub.permute(0, 2, 1, 3) if layout == "bshd" else dq_sub.permute(2, 0, 1, 3)).to(q.dtype)
    return dq, dkn, dv


def det_backward(q, k, v, W, grad_out, causal: bool):
    """Gradients ``(dq, dk, dv)`` of ``det_forward`` (same layouts and dtypes as the inputs)."""
    lib = _lib.load()
    L, B, H, _ = q.shape
    N = v.shape[0]
    qf, kf, vf, gf = _bh(q), _bh(k), _bh(v), _bh(grad_out)
    X = torch.matmul(qf, kf.transpose(-1, -2).contiguous())  # node logits, overwritten by G
    dW = torch.matmul(gf, vf.transpose(-1, -2).contiguous())  # (B, H, L, N)
    with torch.cuda.device(q.device):
        _lib.check(lib.ta_det_grad(X.data_ptr(), N - 1, W.data_ptr(), dW.data_ptr(), N, B * H * L, N,
                                   int(bool(causal)), _stream(q.device)))
    del dW
    G = X
    dq = torch.matmul(G, kf)
    dk = torch.matmul(G.transpose(-1, -2), qf)
    dv = torch.matmul(W.transpose(-1, -2), gf)
    back = lambda t, like: t.permute(2, 0, 1, 3).to(like.dtype)  # noqa: E731
    return back(dq, q), back(dk, k), back(dv, v)


def _edge_forward(q, v):
    """``N <= 1`` outputs of the reference (``_tree_mha.py:367-372``)."""
    if v.shape[0] == 0:
        return torch.zeros_like(q), torch.empty((*q.shape[:-1], 0), device=q.device, dtype=q.dtype)
    return v.expand(q.shape[0], -1, -1, -1).contiguous(), torch.ones((*q.shape[:-1], 1), device=q.device,
                                                                       dtype=q.dtype)


def _edge_backward(q, k, v, grad_out):
    dv = torch.zeros_like(v)
    if v.shape[0] == 1:
        dv[0] = grad_out.float().sum(dim=0).to(v.dtype)
    return torch.zeros_like(q), torch.zeros_like(k), dv


class DeterministicTreeAttention(torch.autograd.Function):
    """Exact tree attention of the reference's ``mode="deterministic"``.

    ``apply(q (L,B,H,D), k (N-1,B,H,D) heap-ordered node keys, v (N,B,H,D),
    is_causal=False) -> (out (L,B,H,D), weights (L,B,H,N) float32)`` with
    ``_deterministic_attention``'s weights (``_tree_mha.py:271-321``): the
    product of the path's sigmoids, or with ``is_causal`` their softmax over
    leaves ``n <= l``.  Gradients ``(dq, dk, dv, None)``; the returned weights
    are not differentiable.  ``N`` must be a power of two.
    """

    @staticmethod
    def forward(ctx, q, k, v, is_causal=False):
        ctx.num_leaves = v.shape[0]
        if v.shape[0] <= 1:
            out, weights = _edge_forward(q, v)
            ctx.save_for_backward(q, k, v)
            ctx.mark_non_differentiable(weights)
            return out, weights
        out, W = det_forward(q, k, v, is_causal)
        ctx.save_for_backward(q, k, v, W)
        ctx.causal = bool(is_causal)
        weights = W.permute(2, 0, 1, 3)
        ctx.mark_non_differentiable(weights)
        return out, weights

    @staticmethod
    def backward(ctx, grad_out, grad_weights):
        del grad_weights
        if ctx.num_leaves <= 1:
            return _edge_backward(*ctx.saved_tensors, grad_out) + (None,)
        q, k, v, W = ctx.saved_tensors
        return det_backward(q, k, v, W, grad_out, ctx.causal) + (None,)


def haar_node_keys(k: torch.Tensor) -> torch.Tensor:
    """Heap-ordered Haar node keys ``(N-1, B, H, D)`` float32 of bshd keys ``k (B, N, H, D)``,
    what the reference adapter feeds the op (``_treeattn_common.py:54-86``, read in heap order)."""
    _on_device(k)
    lib = _lib.load()
    B, N, H, D = k.shape
    k = _prep(k)
    out = torch.empty((N - 1, B, H, D), device=k.device, dtype=torch.float32)
    ks = (ctypes.c_int64 * 3)(*_strides(k, "bshd"))
    nbytes = ctypes.c_int64(0)
    _lib.check(lib.ta_haar_workspace_bytes(B, H, D, N, ctypes.byref(nbytes)))
    work = torch.empty(nbytes.value // 4, device=k.device, dtype=torch.float32)
    with torch.cuda.device(k.device):
        _lib.check(lib.ta_haar_keys(_DTYPES[k.dtype], k.data_ptr(), ks, out.data_ptr(), work.data_ptr(), B, H, D, N,
                                    _stream(k.device)))
    return out


def haar_node_keys_adjoint(dkey: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    """``dk (B, N, H, D)`` in ``like``'s dtype from node-key gradients ``dkey (N-1, B, H, D)``."""
    lib = _lib.load()
    B, N, H, D = like.shape
    dk = torch.empty((B, N, H, D), device=like.device, dtype=like.dtype)
    ks = (ctypes.c_int64 * 3)(*_strides(dk, "bshd"))
    dkey = dkey.float().contiguous()
    with torch.cuda.device(like.device):
        _lib.check(lib.ta_haar_keys_adjoint(_DTYPES[like.dtype], dkey.data_ptr(), dk.data_ptr(), ks, B, H, D, N,
                                            _stream(like.device)))
    return dk


class DeterministicAdapterAttention(torch.autograd.Function):
    """The attn-bench adapter's deterministic path (``baselines/treeattn_torch.py:48-90`` with
    ``TREEATTN_NUM_SAMPLES`` unset): bshd ``q, k, v (B, S, H, D)``, Haar node keys of ``k``,
    exact tree attention; ``apply(q, k, v, causal) -> out (B, S, H, D)``."""

    @staticmethod
    def forward(ctx, q, k, v, causal):
        kt = haar_node_keys(k)
        ctx.causal = bool(causal)
        if det_stream_supported(q, k.shape[1]):
            # 16-bit inputs: streaming forward and backward, nothing of size L x N
            kt = kt.to(q.dtype)
            out, lse = det_stream_forward(q, kt, v, causal, return_lse=True)
            ctx.stream = True
            ctx.save_for_backward(q, k, v, kt, out, *([lse] if lse is not None else []))
            return out
        ctx.stream = False
        ql, vl = q.permute(1, 0, 2, 3), v.permute(1, 0, 2, 3)
        out, W = det_forward(ql, kt, vl, causal)
        ctx.save_for_backward(q, k, v, kt, W)
        return out.permute(1, 0, 2, 3).contiguous()

    @staticmethod
    def backward(ctx, grad_out):
        if ctx.stream:
            q, k, v, kt, out, *lse = ctx.saved_tensors
            dq, dkt, dv = det_stream_backward(q, kt, v, grad_out, out, lse[0] if lse else None, ctx.causal)
            return dq, haar_node_keys_adjoint(dkt, k), dv, None
        q, k, v, kt, W = ctx.saved_tensors
        ql, vl = q.permute(1, 0, 2, 3), v.permute(1, 0, 2, 3)
        dq, dkt, dv = det_backward(ql, kt, vl, W, grad_out.permute(1, 0, 2, 3), ctx.causal)
        dk = haar_node_keys_adjoint(dkt, k)
        return dq.permute(1, 0, 2, 3), dk, dv.permute(1, 0, 2, 3), None


def record_views(q, k, v, opts: TreeOptions, record: torch.Tensor):
    """``(leaves (B,L,H,S) int32, summaries (B*H, NS, D) float32)`` views of a record
    (``D`` padded to a kernel head size where the forward padded it)."""
    if q.shape[-1] not in _HEAD_DIMS:
        q, k, v, opts = _pad_heads(q, k, v, opts)
    q, k, v = _prep(q), _prep(k), _prep(v)
    prob = make_problem(q, k, v, opts)
    lo = _lib.record_offset(prob, _lib.TA_REC_LEAVES)
    so = _lib.record_offset(prob, _lib.TA_REC_SUMMARIES)
    ns = _lib.record_offset(prob, _lib.TA_REC_NUM_ROWS)
    n_leaf = prob.B * prob.L * prob.H * prob.num_samples
    leaves = record[lo:lo + 4 * n_leaf].view(torch.int32).view(prob.B, prob.L, prob.H, prob.num_samples)
    n_sum = prob.B * prob.H * ns * prob.D
    summaries = record[so:so + 4 * n_sum].view(torch.float32).view(prob.B * prob.H, ns, prob.D)
    return leaves, summaries


# ---------------------------------------------------------------------------
# Packed path record (_autograd.py:68-90,179-216): per (position, batch, head,
# sample) the root-to-leaf directions, bit p (p = 0 at the root) in byte p//8
# at bit p%8; in a b-ary tree each level's digit takes log2(b) bits, high bit
# first, so the bits spell the leaf block id most-significant bit first.


def path_bytes(num_leaf_blocks: int) -> int:
    """Bytes per packed path, ``ceil(log2(num_leaf_blocks) / 8)`` (``_autograd.py:68-70``)."""
    out = ctypes.c_int64(0)
    _lib.check(_lib.load().ta_path_bytes(int(num_leaf_blocks), ctypes.byref(out)))
    return out.value


def pack_paths(leaves: torch.Tensor, num_leaf_blocks: int, layout: str = "lbhs") -> torch.Tensor:
    """Leaf block ids (int32, 4-D; dims ordered as ``layout``, ``"lbhs"`` (the
    reference's ``current_nodes``) or ``"blhs"`` (the record's leaves)) ->
    packed paths ``(L, B, H, S, path_bytes)`` uint8."""
    if leaves.dtype != torch.int32 or leaves.dim() != 4 or not leaves.is_cuda:
        raise ValueError("leaves must be a 4-D int32 GPU tensor")
    if layout not in ("lbhs", "blhs"):
        raise ValueError(f"layout must be 'lbhs' or 'blhs', got {layout!r}")
    if layout == "lbhs":
        L, B, H, S = leaves.shape
        st = leaves.stride()
        strides = (st[1], st[0], st[2], st[3])
    else:
        B, L, H, S = leaves.shape
        strides = leaves.stride()
    nb = path_bytes(num_leaf_blocks)
    out = torch.empty((L, B, H, S, nb), device=leaves.device, dtype=torch.uint8)
    st4 = (ctypes.c_int64 * 4)(*strides)
    with torch.cuda.device(leaves.device):
        _lib.check(_lib.load().ta_pack_paths(leaves.data_ptr(), st4, B, L, H, S, int(num_leaf_blocks),
                                              out.data_ptr(), _stream(leaves.device)))
    return out


def unpack_paths(packed: torch.Tensor, num_leaf_blocks: int) -> torch.Tensor:
    """Packed paths ``(L, B, H, S, path_bytes)`` uint8 -> leaf block ids ``(L, B, H, S)`` int32."""
    nb = path_bytes(num_leaf_blocks)
    if packed.dtype != torch.uint8 or packed.dim() != 5 or packed.shape[4] != nb or not packed.is_cuda:
        raise ValueError(f"packed must be a (L, B, H, S, {nb}) uint8 GPU tensor")
    packed = packed.contiguous()
    L, B, H, S, _ = packed.shape
    leaves = torch.empty((L, B, H, S), device=packed.device, dtype=torch.int32)
    st = leaves.stride()
    st4 = (ctypes.c_int64 * 4)(st[1], st[0], st[2], st[3])
    with torch.cuda.device(packed.device):
        _lib.check(_lib.load().ta_unpack_paths(packed.data_ptr(), B, L, H, S, int(num_leaf_blocks),
                                                leaves.data_ptr(), st4, _stream(packed.device)))
    return leaves
