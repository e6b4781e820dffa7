"""CPU tests of the packed path record (``_autograd.py:68-90,179-216``).

* The oracle's ``pack_paths`` is pinned against the reference's heap walk
  (``node <- 2 node + 1 + dir``, leaf ``= node - K``): random directions are
  packed depth by depth the way the reference's sampler does it and must equal
  ``pack_paths`` of the walk's leaf; a pack that wrote the id's bits
  least-significant first, or the bytes in the other order, fails it.
* Round trips, the byte count of ``_path_bit_bytes`` and the b-ary digits.
* The C entry points validate their arguments before launching anything.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import tree_oracle as O
from treeattention_amd import _lib


def _depthwise_pack(dirs: np.ndarray) -> np.ndarray:
    """Pack per-depth directions as the reference's sampler does: byte d//8 |= dir << d%8."""
    T = dirs.shape[-1]
    out = np.zeros(dirs.shape[:-1] + ((T + 7) // 8,), dtype=np.uint8)
    for d in range(T):
        out[..., d // 8] |= (dirs[..., d].astype(np.uint8) << (d % 8))
    return out


@pytest.mark.parametrize("T", [1, 3, 7, 8, 9, 16, 17, 24])
def test_pack_matches_the_reference_walk(T):
    rng = np.random.default_rng(T)
    dirs = rng.integers(0, 2, size=(5, 2, 3, 4, T))
    leaf = O.heap_walk(dirs)
    assert leaf.min() >= 0 and leaf.max() < 2 ** T
    nl = 2 ** T
    assert np.array_equal(O.pack_paths(leaf, nl), _depthwise_pack(dirs))
    assert np.array_equal(O.unpack_paths(O.pack_paths(leaf, nl), nl), leaf)


def test_planted_bit_order_mistake_is_caught():
    rng = np.random.default_rng(0)
    dirs = rng.integers(0, 2, size=(64, 10))
    leaf = O.heap_walk(dirs)
    wrong = np.zeros((64, 2), dtype=np.uint8)
    for p in range(10):  # least-significant id bit first: the mistake a pack could make
        wrong[:, p // 8] |= (((leaf >> p) & 1) << (p % 8)).astype(np.uint8)
    assert not np.array_equal(wrong, _depthwise_pack(dirs))
    assert np.array_equal(O.pack_paths(leaf, 1024), _depthwise_pack(dirs))


def test_path_bytes_is_the_reference_count():
    for nl, nb in [(1, 0), (2, 1), (256, 1), (512, 2), (65536, 2), (131072, 3), (2 ** 24, 3), (2 ** 25, 4)]:
        assert O.path_bytes(nl) == nb
        out = ctypes.c_int64(-1)
        assert _lib.load().ta_path_bytes(nl, ctypes.byref(out)) == 0 and out.value == nb


def test_bary_digits_take_log2b_bits_high_first():
    # b = 4, T = 3 levels: digits j_d, leaf = sum j_d 4^(T-1-d); bits (2d, 2d+1) = (high, low) of j_d
    rng = np.random.default_rng(1)
    digits = rng.integers(0, 4, size=(100, 3))
    leaf = (digits * 4 ** np.arange(2, -1, -1)).sum(-1)
    bits = np.stack([digits >> 1, digits & 1], -1).reshape(100, 6)
    assert np.array_equal(O.pack_paths(leaf, 64), _depthwise_pack(bits))


def test_entry_points_validate_before_launching():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    out = ctypes.c_int64(0)
    assert lib.ta_path_bytes(12, ctypes.byref(out)) == _lib.TA_ERR_INVALID  # not a power of two
    assert b"power of two" in lib.ta_last_error()
    assert lib.ta_pack_paths(None, st, 1, 1, 1, 1, 12, None, None) == _lib.TA_ERR_INVALID
    assert lib.ta_pack_paths(None, st, 1, 1, 1, 1, 16, None, None) == _lib.TA_ERR_INVALID  # NULL pointers
    assert lib.ta_pack_paths(None, st, 0, 4, 4, 4, 16, None, None) == _lib.TA_OK  # nothing to pack
    assert lib.ta_unpack_paths(None, 1, -1, 1, 1, 16, None, st, None) == _lib.TA_ERR_INVALID
    p = _lib.Problem()
    for k_, v_ in dict(B=1, L=64, H=1, D=64, N=64, num_samples=4, branching=2, leaf_block=1,
                       tree_mode=_lib.TA_TREE_COMPAT, causal=_lib.TA_CAUSAL_EXACT, dtype=_lib.TA_BF16,
                       scale=0.125, max_logit=1e3).items():
        setattr(p, k_, v_)
    for a in ("q_strides", "k_strides", "v_strides", "o_strides", "g_strides", "w_strides"):
        getattr(p, a)[:] = (64 * 64, 64, 64)
    assert lib.ta_replay(ctypes.byref(p), None, None, None, None, None) == _lib.TA_ERR_UNSUPPORTED  # causal
    assert b"non-causal" in lib.ta_last_error()
