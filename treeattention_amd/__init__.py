"""MI355X (gfx950) tree attention: hand-written HIP kernels behind a C ABI.

Entry points mirror the reference interfaces: ``hierarchical_attention``
(treeattn-torch / treeattn-cuda op, stochastic and deterministic modes),
``StochasticTreeAttention`` / ``DeterministicTreeAttention`` (autograd
Functions), ``attn_fn`` / ``adapter`` (attn-bench kernel contract), plus
``tree_attention`` for the generalized tree (branching, leaf blocks), and
``pack_paths`` / ``unpack_paths`` for the reference's packed path record.
"""

from .api import (
    KernelAdapter,
    adapter,
    attn_fn,
    hierarchical_attention,
    resolve_num_samples,
    resolve_tree_config,
    tree_attention,
)
from .function import (
    DeterministicTreeAttention,
    StochasticTreeAttention,
    TreeAttentionFunction,
    TreeOptions,
    pack_paths,
    path_bytes,
    tree_backward,
    tree_forward,
    unpack_paths,
)

__all__ = [
    "DeterministicTreeAttention",
    "KernelAdapter",
    "StochasticTreeAttention",
    "TreeAttentionFunction",
    "TreeOptions",
    "adapter",
    "attn_fn",
    "hierarchical_attention",
    "pack_paths",
    "path_bytes",
    "resolve_num_samples",
    "resolve_tree_config",
    "tree_attention",
    "tree_backward",
    "tree_forward",
    "unpack_paths",
]
