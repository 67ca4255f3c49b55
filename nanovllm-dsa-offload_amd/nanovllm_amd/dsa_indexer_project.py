"""DSA indexer projection on MI355X: the producer of the LIM inputs.

Mirrors the two public functions of the reference module
nanovllm/models/dsa_indexer_project.py (same names, arguments, output
buffers and ``ValueError`` conditions):

* :func:`dsa_indexer_project_query_only` (reference :296-355), the stable
  decode path: ``q_index = RoPE(q_c . wq_b^T)`` and
  ``index_weights = hidden . weights_proj^T * score_scale``.  When
  ``weights_proj_weight`` shares the activations' dtype (the decode graph's
  cached low-precision copy, nanovllm/models/glm_mla.py:262-271) both come
  from one fused gfx950 launch (``nvdsa_dsa_indexer_project_query_only``).
  Otherwise q comes from that launch and the weights from an fp32 library
  GEMM then one cast, as the reference computes them (:82-86).
  ``wq_b_bmm_t`` / ``enable_q_bmm`` are accepted for signature parity; the
  fused kernel reads ``wq_b_weight`` in its natural [H*D, R] layout, so the
  transposed BMM copy (an Ascend layout, :102-130) is not used.
* :func:`dsa_indexer_project` (reference :245-293), the prefill path: q as
  above, ``index_k = RoPE(LayerNorm(hidden . wk^T))`` and fp32 weights.  The
  k projection and layer norm are library calls; both RoPEs are the HIP
  kernel behind ``torch.ops.nanovllm_dsa.dsa_indexer_query_rope_inplace``.

RoPE is the interleaved-pair rotation of the reference's AscendC kernel
(ops/dsa_indexer_project/op_kernel/dsa_indexer_project_kernel.cpp:105-176):
fp32 products and sum, rounded once to the 16-bit dtype.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops


def _check_project_outputs(q_index_out, index_k_out, index_weights_out, *, num_tokens, n_head, head_dim, dtype,
                           device) -> None:
    """The reference's output checks (dsa_indexer_project.py:135-155)."""
    if q_index_out.shape != (num_tokens, n_head, head_dim):
        raise ValueError(f"q_index_out shape must be {(num_tokens, n_head, head_dim)}, got {tuple(q_index_out.shape)}")
    if index_k_out.shape != (num_tokens, head_dim):
        raise ValueError(f"index_k_out shape must be {(num_tokens, head_dim)}, got {tuple(index_k_out.shape)}")
    if index_weights_out.shape != (num_tokens, n_head):
        raise ValueError(f"index_weights_out shape must be {(num_tokens, n_head)}, got {tuple(index_weights_out.shape)}")
    for name, tensor in (("q_index_out", q_index_out), ("index_k_out", index_k_out),
                         ("index_weights_out", index_weights_out)):
        if tensor.dtype != dtype or tensor.device != device:
            raise ValueError(f"{name} must use dtype={dtype} and device={device}, got dtype={tensor.dtype} "
                             f"device={tensor.device}")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")


def _rope_cos_sin(cos: torch.Tensor, sin: torch.Tensor, tokens: int, rope_dim: int):
    """cos/sin as the [T, 1, 1, rope_dim] tensors the RoPE op reads (the
    reference's reshape(T, -1)[..., :rope_dim], :28-32)."""
    c = cos.reshape(tokens, -1)[..., :rope_dim].contiguous().view(tokens, 1, 1, rope_dim)
    s = sin.reshape(tokens, -1)[..., :rope_dim].contiguous().view(tokens, 1, 1, rope_dim)
    return c, s


def _weights_fp32(hidden_states, weights_proj_weight, score_scale: float) -> torch.Tensor:
    """Reference :82-86 (dtype mismatch): fp32 projection, scale, one cast."""
    weights = F.linear(hidden_states.float(), weights_proj_weight.float())
    if float(score_scale) != 1.0:
        weights = weights * float(score_scale)
    return weights.to(hidden_states.dtype)


def dsa_indexer_project_query_only(hidden_states, q_c, cos, sin, wq_b_weight, weights_proj_weight, q_index_out,
                                   index_weights_out, *, n_head, head_dim, rope_dim, score_scale, wq_b_bmm_t=None,
                                   enable_q_bmm=False):
    """Decode-only indexer projection (reference dsa_indexer_project.py:296-355)."""
    del wq_b_bmm_t, enable_q_bmm  # the fused kernel reads wq_b_weight directly
    if q_index_out.shape != (hidden_states.shape[0], n_head, head_dim):
        raise ValueError(f"q_index_out shape must be {(hidden_states.shape[0], n_head, head_dim)}, "
                         f"got {tuple(q_index_out.shape)}")
    if index_weights_out.shape != (hidden_states.shape[0], n_head):
        raise ValueError(f"index_weights_out shape must be {(hidden_states.shape[0], n_head)}, "
                         f"got {tuple(index_weights_out.shape)}")
    same = weights_proj_weight.dtype == hidden_states.dtype
    ops.indexer_project_query_only(hidden_states, q_c, cos, sin, wq_b_weight, weights_proj_weight if same else None,
                                   q_index_out, index_weights_out if same else None, n_head, head_dim, rope_dim,
                                   score_scale)
    if not same:
        index_weights_out.copy_(_weights_fp32(hidden_states, weights_proj_weight, score_scale))
    return q_index_out, index_weights_out


def dsa_indexer_project(hidden_states, q_c, cos, sin, wq_b_weight, wk_weight, k_norm_weight, k_norm_bias,
                        weights_proj_weight, q_index_out, index_k_out, index_weights_out, *, n_head, head_dim,
                        rope_dim, score_scale, wq_b_bmm_t=None, enable_q_bmm=False):
    """Prefill indexer projection (reference dsa_indexer_project.py:245-293)."""
    del wq_b_bmm_t, enable_q_bmm
    tokens = int(hidden_states.shape[0])
    _check_project_outputs(q_index_out, index_k_out, index_weights_out, num_tokens=tokens, n_head=int(n_head),
                           head_dim=int(head_dim), dtype=hidden_states.dtype, device=hidden_states.device)
    # q: projection + RoPE in one launch (no weights part).
    ops.indexer_project_query_only(hidden_states, q_c, cos, sin, wq_b_weight, None, q_index_out, None, n_head,
                                   head_dim, rope_dim, 1.0)
    # k: library projection and layer norm, then the RoPE kernel on [T, 1, D].
    k = F.linear(hidden_states, wk_weight)
    k = F.layer_norm(k, (int(head_dim),), k_norm_weight, k_norm_bias, eps=1e-6)
    index_k_out.copy_(k)
    if tokens:
        c, s = _rope_cos_sin(cos, sin, tokens, int(rope_dim))
        ops.dsa_indexer_query_rope_inplace(index_k_out.view(tokens, 1, int(head_dim)), c, s, int(rope_dim))
    index_weights_out.copy_(_weights_fp32(hidden_states, weights_proj_weight, score_scale))
    return q_index_out, index_k_out, index_weights_out


__all__ = ["dsa_indexer_project", "dsa_indexer_project_query_only"]
