"""Writes golden vectors of the reference's stochastic and deterministic tree attention.

Runs the reference's own pure-PyTorch implementation
(``packages/treeattn-torch/src/treeattn_torch/_tree_mha.py``) in THIS container,
imported read-only from ``/root/reference`` (no bytecode is written there), on
tiny seeded inputs, and stores inputs and outputs as ``.npz`` fixtures next to
this script.  The reference draws its Gumbel noise with
``torch.Tensor.exponential_`` (``_tree_mha.py:109,255``); this script replaces
that method, for the duration of each call, by one that fills the tensor with
``E = -log(u)`` from the uniform tensor ``U`` (B, L, H, S, T, 2) that the
backend under test consumes, in the order the reference draws them:

* non-causal sampler: one (L, B, H, S, 2) draw per depth d -> U[:, :, :, :, d, :];
* causal sampler: one (B, H, S, 2) draw per query t (absolute position) and
  depth d -> U[:, t, :, :, d, :].

Fixture keys: inputs ``q, k, v`` (op-level (L, B, H, D) / (K, B, H, D) /
(N, B, H, D) layouts, heap-ordered node keys), ``dout``, ``U``; reference
results ``out`` (L, B, E), ``weights``, ``dq, dk, dv`` (autograd of
``<dout, out>``), and where the sampler is called directly ``idx`` / ``lp``.

Usage (needs /root/reference; not run by the tests):
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

sys.dont_write_bytecode = True
os.environ["PYTHONDONTWRITEBYTECODE"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
REF_SRC = "/root/reference/packages/treeattn-torch/src"

from oracle import tree_oracle as O  # noqa: E402


def _import_reference():
    sys.path.insert(0, REF_SRC)
    from treeattn_torch import _tree_mha  # noqa: F401

    return _tree_mha


class NoiseFromUniforms:
    """Context manager: ``exponential_`` fills from U in the reference's draw order."""

    def __init__(self, U: np.ndarray, plan: list[tuple[tuple[int, ...], np.ndarray]]):
        self.plan = list(plan)
        self.U = U

    def __enter__(self):
        self.orig = torch.Tensor.exponential_
        plan = self.plan

        def fill(t, *args, **kwargs):
            shape, E = plan.pop(0)
            assert tuple(t.shape) == tuple(shape), (tuple(t.shape), shape)
            with torch.no_grad():
                t.copy_(torch.from_numpy(E).to(t.dtype))
            return t

        torch.Tensor.exponential_ = fill
        return self

    def __exit__(self, *exc):
        torch.Tensor.exponential_ = self.orig
        assert not self.plan or exc[0] is not None, f"{len(self.plan)} noise draws unused"
        return False


def noncausal_plan(U):
    B, L, H, S, T, _ = U.shape
    E = -np.log(U.astype(np.float64))
    return [((L, B, H, S, 2), np.ascontiguousarray(E[:, :, :, :, d, :].transpose(1, 0, 2, 3, 4))) for d in range(T)]


def causal_plan(U, t0):
    B, L, H, S, T, _ = U.shape
    E = -np.log(U.astype(np.float64))
    return [((B, H, S, 2), np.ascontiguousarray(E[:, t, :, :, d, :])) for t in range(t0, L) for d in range(T)]


def make_case(ref, name, L, B, H, D, S, causal, dtype, seed, mode="stochastic"):
    N = L
    T = (N - 1).bit_length()
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(L, B, H, D, generator=g)
    k = torch.randn(N - 1, B, H, D, generator=g) * 0.5
    v = torch.randn(N, B, H, D, generator=g)
    dout = torch.randn(L, B, H * D, generator=g)
    U = O.uniforms(seed, (B, L, H, S, T, 2))
    qr, kr, vr = (x.to(dtype).reshape(x.shape[0], B, H * D).requires_grad_(True) for x in (q, k, v))
    plan = []
    if mode == "stochastic":
        if causal and L > S:
            plan = causal_plan(U, S)
        elif causal:
            plan = causal_plan(U, 0)
        else:
            plan = noncausal_plan(U)
    with NoiseFromUniforms(U, plan):
        out, weights = ref.hierarchical_attention(qr, kr, vr, num_heads=H, is_causal=causal, mode=mode,
                                                  num_samples=S)
    out.backward(dout.to(dtype))
    res = dict(q=q.to(dtype).float().numpy(), k=k.to(dtype).float().numpy(), v=v.to(dtype).float().numpy(),
               dout=dout.to(dtype).float().numpy(), U=U, out=out.detach().float().numpy(),
               weights=weights.detach().float().numpy(), dq=qr.grad.float().numpy(), dk=kr.grad.float().numpy(),
               dv=vr.grad.float().numpy(), L=L, B=B, H=H, D=D, S=S, causal=int(causal),
               dtype=str(dtype).replace("torch.", ""), mode=mode)
    # sampled indices straight from the reference samplers (same noise)
    if mode == "stochastic":
        qh = q.to(dtype)
        kh = k.to(dtype)
        with torch.no_grad():
            if causal:
                t0 = S if L > S else 0
                with NoiseFromUniforms(U, causal_plan(U, t0)):
                    idx, lp = ref._sample_paths_causal(qh[t0:], kh, S, N, causal_offset=t0)
            else:
                with NoiseFromUniforms(U, noncausal_plan(U)):
                    idx, lp = ref._sample_paths_non_causal(qh, kh, S, N)
        res.update(idx=idx.numpy(), lp=lp.float().numpy())
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **res)
    print(f"wrote {name}.npz: out {tuple(out.shape)} weights {tuple(weights.shape)}")


def main():
    ref = _import_reference()
    f32, bf16 = torch.float32, torch.bfloat16
    cases = [
        # name, L, B, H, D, S, causal, dtype, seed
        ("noncausal_f32_L16", 16, 1, 2, 16, 4, False, f32, 1),
        ("noncausal_f32_L32", 32, 2, 2, 16, 4, False, f32, 2),
        ("noncausal_bf16_L32", 32, 1, 2, 32, 8, False, bf16, 3),
        ("causal_hybrid_f32_L32", 32, 2, 2, 16, 4, True, f32, 4),
        ("causal_hybrid_f32_L64", 64, 1, 4, 16, 8, True, f32, 5),
        ("causal_short_f32_L8", 8, 1, 2, 16, 8, True, f32, 6),
        ("causal_hybrid_bf16_L32", 32, 1, 2, 32, 4, True, bf16, 7),
    ]
    for c in cases:
        make_case(ref, *c)
    make_case(ref, "deterministic_causal_f32_L16", 16, 1, 2, 16, 4, True, f32, 8, mode="deterministic")
    make_case(ref, "deterministic_noncausal_f32_L16", 16, 1, 2, 16, 4, False, f32, 9, mode="deterministic")


if __name__ == "__main__":
    main()
