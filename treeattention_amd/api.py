"""Public entry points with the reference's interfaces.

* ``hierarchical_attention`` -- same signature, shapes and errors as
  treeattn-torch / treeattn-cuda (``_tree_mha.py:324-413``,
  ``_autograd.py:863-915``): ``query (L,B,E)``, ``key (N-1,B,E)`` heap-ordered
  node keys, ``value (N,B,E)`` -> ``(out (L,B,E), weights (L,B,H,S))``.
* ``tree_attention`` -- bshd tensors with the generalized tree (branching,
  leaf block, summaries built from the keys).
* ``attn_fn`` / ``adapter`` -- attn-bench's kernel contract
  (``adapters.py:29-58``): ``fn(q, k, v, causal, softmax_scale)`` on
  ``(B, S, H, D)`` tensors, no in-place writes, deterministic forward, no
  host syncs.  Configured like the reference adapters through environment
  variables (``_treeattn_common.py:27-47``).
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Callable

import torch

from .function import (
    DeterministicAdapterAttention,
    DeterministicTreeAttention,
    StochasticTreeAttention,
    TreeAttentionFunction,
    TreeOptions,
)

NUM_SAMPLES_ENV_VAR = "TREEATTN_NUM_SAMPLES"
BRANCHING_ENV_VAR = "TREEATTN_BRANCHING"
LEAF_BLOCK_ENV_VAR = "TREEATTN_LEAF_BLOCK"
TREE_MODE_ENV_VAR = "TREEATTN_TREE_MODE"
SEED_ENV_VAR = "TREEATTN_SEED"

_DEFAULT_BLOCK_SIZE = 256
_DEFAULT_MAX_LOGIT = 1e3


def resolve_num_samples() -> int | None:
    """``num_samples`` from ``TREEATTN_NUM_SAMPLES``; ``None`` means deterministic mode.

    Same parsing as ``_treeattn_common.py:30-47``: unset, empty or ``"0"`` ->
    ``None``; a non-integer or a negative value raises ``ValueError``.
    """
    raw = os.environ.get(NUM_SAMPLES_ENV_VAR, "").strip()
    if not raw or raw == "0":
        return None
    try:
        n = int(raw)
    except ValueError as e:
        raise ValueError(f"{NUM_SAMPLES_ENV_VAR}={raw!r} is not an integer") from e
    if n < 0:
        raise ValueError(f"{NUM_SAMPLES_ENV_VAR}={n} must be >= 0")
    return n or None


def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name, "").strip()
    if not raw:
        return default
    try:
        return int(raw)
    except ValueError as e:
        raise ValueError(f"{name}={raw!r} is not an integer") from e


def resolve_tree_config() -> dict:
    """Tree shape for the adapter: branching, leaf block, summary mode, seed.

    Defaults (``2, 1, "compat", 0``) are the reference's tree: binary, one
    token per leaf, Haar keys in the reference layout.
    """
    mode = os.environ.get(TREE_MODE_ENV_VAR, "").strip() or "compat"
    if mode not in ("compat", "natural"):
        raise ValueError(f"{TREE_MODE_ENV_VAR}={mode!r} must be 'compat' or 'natural'")
    return dict(
        branching=_env_int(BRANCHING_ENV_VAR, 2),
        leaf_block=_env_int(LEAF_BLOCK_ENV_VAR, 1),
        tree_mode=mode,
        seed=_env_int(SEED_ENV_VAR, 0),
    )


def hierarchical_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    num_heads: int,
    is_causal: bool = False,
    mode: str = "stochastic",
    num_samples: int = 64,
    *,
    block_size: int = _DEFAULT_BLOCK_SIZE,
    max_logit: float = _DEFAULT_MAX_LOGIT,
    seed: int = 0,
    uniforms: torch.Tensor | None = None,
    paths: torch.Tensor | None = None,
    return_paths: bool = False,
):
    """Hierarchical attention, reference signature (``_tree_mha.py:324-413``).

    ``mode="stochastic"``: ``uniforms`` (optional, float32 ``(B, L, H, S, T,
    2)``, contiguous) replaces the Gumbel noise stream; without it the counter
    RNG with ``seed`` supplies it, so equal inputs give equal outputs.
    ``paths`` (optional, non-causal): the reference's packed path record
    ``(L, B, H, S, ceil(log2(N)/8))`` uint8 (``_autograd.py:68-90``) to replay
    instead of sampling; ``return_paths=True`` returns ``(out, weights,
    packed_paths)`` with the forward's own paths in that format.
    ``mode="deterministic"``: exact attention over every leaf, weights
    ``(L, B, H, N)`` (``_tree_mha.py:271-321``); ``N`` a power of two.
    """
    if mode not in ("stochastic", "deterministic"):
        raise ValueError(f"mode must be 'stochastic' or 'deterministic', got {mode!r}")
    if mode == "stochastic" and num_samples is None:
        raise ValueError("num_samples must be provided for stochastic mode.")
    if query.dim() != 3 or value.dim() != 3:
        raise ValueError("query and value must have shape (L, B, E) and (N, B, E)")
    L, B, E = query.shape
    N = value.shape[0]
    H = num_heads
    if E % H != 0:
        raise ValueError(f"embed_dim={E} is not divisible by num_heads={H}")
    D = E // H
    K = N - 1
    if K > 0 and key.shape[0] != K:
        raise ValueError(f"Key tensor length must be N-1 ({K}), but got {key.shape[0]}.")
    q = query.reshape(L, B, H, D)
    k = key.reshape(max(K, 0), B, H, D) if K > 0 else key.new_empty((0, B, H, D))
    v = value.reshape(N, B, H, D)
    if mode == "deterministic":
        if paths is not None or return_paths:
            raise ValueError("paths / return_paths apply to mode='stochastic'")
        out, weights = DeterministicTreeAttention.apply(q, k, v, bool(is_causal))
        return out.reshape(L, B, E), weights
    res = StochasticTreeAttention.apply(q, k, v, num_samples, block_size, max_logit, is_causal, seed, uniforms, paths,
                                        bool(return_paths))
    return (res[0].reshape(L, B, E),) + tuple(res[1:])


def tree_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    *,
    num_samples: int,
    branching: int = 2,
    leaf_block: int = 1,
    tree_mode: str = "compat",
    seed: int = 0,
    max_logit: float = _DEFAULT_MAX_LOGIT,
    uniforms: torch.Tensor | None = None,
    return_weights: bool = False,
    causal_mode: str = "auto",
    paths: torch.Tensor | None = None,
    dense_cols: int = 0,
):
    """Stochastic tree attention on ``(B, L, H, D)`` tensors.

    The keys are pooled into per-node child summaries (``tree_mode``), each
    query samples ``num_samples`` root-to-leaf paths with Gumbel-max
    decisions, and the output is ``sum_s w_s softmax(scale q K_blk^T) V_blk``
    with ``w = softmax`` of the sampled path log-probabilities.  With
    ``branching=2, leaf_block=1, tree_mode="compat"`` this is the reference
    adapter's stochastic computation (``baselines/treeattn_torch.py:48-90``),
    causal included (``causal_mode="auto"`` selects the reference's causal
    semantics on that tree; see ``TreeOptions``).  ``paths`` (non-causal):
    packed path bits ``(L, B, H, S, path_bytes(L // leaf_block))`` uint8 to
    replay instead of sampling (``pack_paths``).  ``dense_cols``: see ``TreeOptions`` (tuning).
    """
    opts = TreeOptions(num_samples=int(num_samples), branching=int(branching), leaf_block=int(leaf_block),
                       tree_mode=tree_mode, causal=bool(causal), causal_mode=causal_mode, scale=softmax_scale,
                       max_logit=float(max_logit), seed=int(seed), layout="bshd", dense_cols=int(dense_cols))
    out, weights = TreeAttentionFunction.apply(q, k, v, opts, uniforms, paths)
    return (out, weights) if return_weights else out


def attn_fn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, softmax_scale: float | None) -> torch.Tensor:
    """attn-bench kernel: ``(B, S, H, D)`` in, same shape and dtype out.

    Like treeattn-torch's adapter (``baselines/treeattn_torch.py:48-90``):
    ``TREEATTN_NUM_SAMPLES`` set -> stochastic mode with that many paths,
    unset (or ``0``) -> deterministic (exact) mode on the reference tree (Haar
    node keys of ``k``, ``S`` a power of two).  The stochastic tree shape
    comes from ``TREEATTN_BRANCHING`` / ``TREEATTN_LEAF_BLOCK`` /
    ``TREEATTN_TREE_MODE`` (default: the reference tree).  ``softmax_scale``
    is used inside leaf blocks only (the reference ignores it,
    ``baselines/treeattn_torch.py:53``; at ``leaf_block=1`` it has no effect).
    """
    num_samples = resolve_num_samples()
    cfg = resolve_tree_config()
    if num_samples is None:
        if (cfg["branching"], cfg["leaf_block"], cfg["tree_mode"]) != (2, 1, "compat"):
            raise ValueError("deterministic mode (TREEATTN_NUM_SAMPLES unset) runs on the reference tree only: "
                             "branching 2, leaf block 1, compat keys")
        S = q.shape[1]
        if S < 2 or S & (S - 1):
            raise ValueError(f"deterministic tree attention requires power-of-two seqlen, got {S}")
        return DeterministicAdapterAttention.apply(q, k, v, bool(causal))
    return tree_attention(q, k, v, causal, softmax_scale, num_samples=num_samples, **cfg)


@dataclass(frozen=True)
class KernelAdapter:
    """Same fields and compatibility check as attn-bench's ``KernelAdapter`` (``adapters.py:32-58``)."""

    name: str
    fn: Callable
    supports_backward: bool = True
    supports_causal: bool = True
    allowed_dtypes: frozenset = field(default_factory=lambda: frozenset({torch.float16, torch.bfloat16}))
    allowed_head_dims: frozenset = field(default_factory=lambda: frozenset({32, 64, 96, 128}))
    layout: str = "bshd"

    def is_compatible(self, dtype: torch.dtype, head_dim: int, causal: bool) -> tuple[bool, str]:
        if dtype not in self.allowed_dtypes:
            allowed = ", ".join(str(d) for d in sorted(self.allowed_dtypes, key=str))
            return False, f"dtype {dtype} not in allowed_dtypes ({allowed})"
        if head_dim not in self.allowed_head_dims:
            allowed = ", ".join(str(h) for h in sorted(self.allowed_head_dims))
            return False, f"head_dim {head_dim} not in allowed_head_dims ({allowed})"
        if causal and not self.supports_causal:
            return False, "kernel does not support causal=True"
        return True, ""


BASELINE_NAME = "treeattn_mi355x"


def adapter():
    """attn-bench adapter factory (``--kernel treeattention_amd.api:adapter``).

    Returns attn-bench's own ``KernelAdapter`` when that package is
    importable, else the field-compatible local class.
    """
    try:
        from attn_bench.adapters import KernelAdapter as _KA  # type: ignore
    except Exception:  # attn-bench not installed
        _KA = KernelAdapter
    return _KA(
        name=BASELINE_NAME,
        fn=attn_fn,
        supports_backward=True,
        supports_causal=True,
        allowed_dtypes=frozenset({torch.float16, torch.bfloat16, torch.float32}),
        allowed_head_dims=frozenset({32, 64, 96, 128}),
        layout="bshd",
    )
