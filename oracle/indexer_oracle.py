"""CPU oracle of the DSA indexer projection — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
path (``nanovllm_amd``) never imports, calls or falls back to it.

It restates in numpy:

* ``rope_pairs_f32`` / ``query_rope_inplace`` — the interleaved-pair RoPE of
  the reference's AscendC kernel
  (csrc/nanovllm_ascend_ops/ops/dsa_indexer_project/op_kernel/dsa_indexer_project_kernel.cpp:60-176):
  per pair (even, odd) the rotated pair is (-odd, even) (the [odd, even]
  swap times the [-1, +1] sign pair, :118-140), out = x*cos + rotated*sin
  with each product and the sum rounded in fp32 (:149-161), then a
  round-to-nearest-even cast (:162-163).  cos/sin of token t sit at
  t*rope_dim (:76-78).
* ``project_query_only`` — nanovllm/models/dsa_indexer_project.py:296-355:
  q = q_c . wq_b^T rounded to the 16-bit dtype (F.linear, :93-104), then the
  RoPE above on its first rope_dim dims with cos/sin taken as
  reshape(T, -1)[..., :rope_dim] (:28-32); weights = hidden . w_proj^T
  rounded, times score_scale rounded again when the scale is not 1 (same
  dtype, :74-80) or computed in fp32 and rounded once (fp32 w_proj, :82-86).
* ``project_full`` — dsa_indexer_project (:245-293): the q above, k =
  RoPE(LayerNorm(hidden . wk^T), eps 1e-6) and fp32 weights.

The projections are evaluated in float64 and rounded to float32 before the
16-bit rounding (the GPU accumulates in fp32 in another order, so random
inputs compare within a tolerance; one-hot weights make every projection
exact and everything bit-exact).  Pinned by tests/test_indexer_oracle.py:
identity and quarter-turn rotations, a float64 textbook rotation, the
reference test's one-hot projections
(ut_ops/test_glm_dsa_indexer.py:127-192) and its independent RoPE golden
(:99-124).
"""

from __future__ import annotations

import numpy as np

from .dsa_oracle import bits_to_f32, f32_to_bits


def rope_pairs_f32(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Interleaved-pair rotation in float32, every operation rounded."""
    x = np.asarray(x, np.float32)
    cos = np.asarray(cos, np.float32)
    sin = np.asarray(sin, np.float32)
    rotated = np.empty_like(x)
    rotated[..., 0::2] = -x[..., 1::2]
    rotated[..., 1::2] = x[..., 0::2]
    a = np.multiply(x, cos, dtype=np.float32)
    b = np.multiply(rotated, sin, dtype=np.float32)
    return np.add(a, b, dtype=np.float32)


def query_rope_inplace(q_bits: np.ndarray, cos_bits: np.ndarray, sin_bits: np.ndarray, rope_dim: int,
                       dtype: str = "bf16") -> None:
    """The op dsa_indexer_query_rope_inplace: q_bits [T, H, D] (uint16)
    rotated in place on its first rope_dim dims."""
    T = q_bits.shape[0]
    c = bits_to_f32(np.asarray(cos_bits).reshape(-1)[:T * rope_dim], dtype).reshape(T, 1, rope_dim)
    s = bits_to_f32(np.asarray(sin_bits).reshape(-1)[:T * rope_dim], dtype).reshape(T, 1, rope_dim)
    x = bits_to_f32(q_bits[..., :rope_dim], dtype)
    q_bits[..., :rope_dim] = f32_to_bits(rope_pairs_f32(x, c, s), dtype).reshape(x.shape)


def _round16(x64: np.ndarray, dtype: str) -> np.ndarray:
    return f32_to_bits(np.asarray(x64).astype(np.float32), dtype).reshape(np.shape(x64))


def _cos_sin_rows(cos_bits, sin_bits, tokens: int, rope_dim: int, dtype: str):
    c = bits_to_f32(np.asarray(cos_bits).reshape(tokens, -1)[:, :rope_dim], dtype)
    s = bits_to_f32(np.asarray(sin_bits).reshape(tokens, -1)[:, :rope_dim], dtype)
    return c, s


def _q_rows(qc_bits, wq_bits, cos_bits, sin_bits, n_head: int, head_dim: int, rope_dim: int, dtype: str):
    T = qc_bits.shape[0]
    qc = bits_to_f32(qc_bits, dtype).astype(np.float64)
    wq = bits_to_f32(wq_bits, dtype).astype(np.float64)
    q = _round16(qc @ wq.T, dtype).reshape(T, n_head, head_dim)
    c, s = _cos_sin_rows(cos_bits, sin_bits, T, rope_dim, dtype)
    x = bits_to_f32(q[..., :rope_dim], dtype)
    q[..., :rope_dim] = f32_to_bits(rope_pairs_f32(x, c[:, None, :], s[:, None, :]), dtype).reshape(x.shape)
    return q


def project_query_only(hidden_bits, qc_bits, cos_bits, sin_bits, wq_bits, w_proj, n_head: int, head_dim: int,
                       rope_dim: int, score_scale: float, dtype: str = "bf16"):
    """Returns (q_index bits [T, H, D], index_weights bits [T, H]).
    ``w_proj`` is either 16-bit patterns (same dtype as the activations) or
    a float32 array (the reference's fp32 weights_proj)."""
    q = _q_rows(qc_bits, wq_bits, cos_bits, sin_bits, n_head, head_dim, rope_dim, dtype)
    h = bits_to_f32(hidden_bits, dtype).astype(np.float64)
    w_proj = np.asarray(w_proj)
    if w_proj.dtype == np.float32:
        w32 = (h @ w_proj.astype(np.float64).T).astype(np.float32)
        if float(score_scale) != 1.0:
            w32 = np.multiply(w32, np.float32(score_scale), dtype=np.float32)
        return q, f32_to_bits(w32, dtype).reshape(w32.shape)
    w = _round16(h @ bits_to_f32(w_proj, dtype).astype(np.float64).T, dtype)
    if float(score_scale) != 1.0:
        w32 = np.multiply(bits_to_f32(w, dtype), np.float32(score_scale), dtype=np.float32)
        w = f32_to_bits(w32, dtype).reshape(w32.shape)
    return q, w


def project_full(hidden_bits, qc_bits, cos_bits, sin_bits, wq_bits, wk_bits, k_norm_w_bits, k_norm_b_bits,
                 w_proj_f32, n_head: int, head_dim: int, rope_dim: int, score_scale: float, dtype: str = "bf16"):
    """Returns (q_index, index_k, index_weights) bits of the prefill path."""
    T = hidden_bits.shape[0]
    q = _q_rows(qc_bits, wq_bits, cos_bits, sin_bits, n_head, head_dim, rope_dim, dtype)
    h = bits_to_f32(hidden_bits, dtype).astype(np.float64)
    k16 = _round16(h @ bits_to_f32(wk_bits, dtype).astype(np.float64).T, dtype)
    k = bits_to_f32(k16, dtype).astype(np.float64)
    mean = k.mean(axis=-1, keepdims=True)
    var = ((k - mean) ** 2).mean(axis=-1, keepdims=True)
    kn = (k - mean) / np.sqrt(var + 1e-6)
    kn = kn * bits_to_f32(k_norm_w_bits, dtype).astype(np.float64)
    if k_norm_b_bits is not None:
        kn = kn + bits_to_f32(k_norm_b_bits, dtype).astype(np.float64)
    k16 = _round16(kn, dtype)
    c, s = _cos_sin_rows(cos_bits, sin_bits, T, rope_dim, dtype)
    x = bits_to_f32(k16[..., :rope_dim], dtype)
    k16[..., :rope_dim] = f32_to_bits(rope_pairs_f32(x, c, s), dtype).reshape(x.shape)
    w32 = (h @ np.asarray(w_proj_f32, np.float64).T).astype(np.float32)
    w32 = np.multiply(w32, np.float32(score_scale), dtype=np.float32)
    return q, k16, f32_to_bits(w32, dtype).reshape(w32.shape)
