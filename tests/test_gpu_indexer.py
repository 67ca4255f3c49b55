"""Indexer projection and query RoPE on the GPU vs the oracle.

* ``dsa_indexer_query_rope_inplace`` (reference schema, nanovllm_ops.cpp:713-714):
  bit-exact against the oracle's restatement of the AscendC kernel, bf16 and
  fp16, several token / head counts and a smaller rope width.
* ``dsa_indexer_project_query_only``, fused launch: with the reference test's
  one-hot projections (ut_ops/test_glm_dsa_indexer.py:127-192) every
  projection is exact, so q and the weights are bit-exact against the oracle
  (which the CPU tests pin to the closed form), including the score-scale
  rounding and token counts that cross the 64-token groups.  With random
  projections the fp32 accumulation order differs from the oracle's float64
  sums, so the test allows the 16-bit rounding to land a step apart: at
  most 2^-7 (bf16) / 2^-10 (fp16) relative to the value (to the pair's norm
  for rotated dims), and at least 98% (95% rotated) of the values exact.
* the fp32 ``weights_proj`` path and the prefill ``dsa_indexer_project``
  (k through a library layer norm: the reference test's tolerances,
  atol 0.05 / rtol 0.025).
* the reference's argument errors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, dname
from oracle import dsa_oracle as O
from oracle import indexer_oracle as I

pytestmark = pytest.mark.gpu

H, D, R, HID, ROPE = 32, 128, 2048, 6144, 64


def _dev(x_bits: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).view(dtype).to("cuda")


def _to_bits(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    return O.f32_to_bits(np.asarray(x, np.float32), dname(dtype)).reshape(np.shape(x))


def _cos_sin(T, dtype, rope=ROPE, seed=0):
    rng = np.random.default_rng(seed)
    pos = rng.integers(1, 40000, size=(T, 1)).astype(np.float64)
    freq = 10000.0 ** (-np.arange(rope // 2) * 2.0 / rope)
    ang = np.repeat(pos * freq[None, :], 2, axis=1)
    return _to_bits(np.cos(ang), dtype).reshape(T, 1, 1, rope), _to_bits(np.sin(ang), dtype).reshape(T, 1, 1, rope)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,heads,head_dim,rope", [(1, 32, 128, 64), (24, 32, 128, 64), (100, 64, 128, 64),
                                                   (7, 16, 64, 32)])
def test_query_rope_bit_exact(dtype, T, heads, head_dim, rope):
    from nanovllm_amd import ops

    print(f"ROPE {dtype} T={T} H={heads} D={head_dim} rope={rope}", flush=True)
    rng = np.random.default_rng(T + heads)
    q = _to_bits(rng.standard_normal((T, heads, head_dim)) * 3, dtype)
    c, s = _cos_sin(T, dtype, rope, seed=T)
    qd = _dev(q, dtype)
    ops.dsa_indexer_query_rope_inplace(qd, _dev(c, dtype), _dev(s, dtype), rope)
    torch.cuda.synchronize()
    expect = q.copy()
    I.query_rope_inplace(expect, c, s, rope, dname(dtype))
    assert np.array_equal(bits(qd), expect)


def test_query_rope_errors():
    from nanovllm_amd import ops

    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16, device="cuda")
    c = torch.zeros(4, 1, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="aligned to 16"):
        ops.dsa_indexer_query_rope_inplace(q, c, c, 56)
    with pytest.raises(RuntimeError, match="cos dtype mismatch"):
        ops.dsa_indexer_query_rope_inplace(q, c.half(), c, 64)
    with pytest.raises(RuntimeError, match="token dimension mismatch"):
        ops.dsa_indexer_query_rope_inplace(q, c[:3], c[:3], 64)


def _one_hot():
    q_rows = H * D
    wq = np.zeros((q_rows, R), np.float32)
    wq[np.arange(q_rows), (np.arange(q_rows) * 17 + 11) % R] = np.where(np.arange(q_rows) % 3 == 0, -1.0, 1.0)
    wp = np.zeros((H, HID), np.float32)
    wp[np.arange(H), (np.arange(H) * 43 + 5) % HID] = np.where(np.arange(H) % 2 == 0, 1.0, -1.0)
    wk = np.zeros((D, HID), np.float32)
    wk[np.arange(D), (np.arange(D) * 29 + 7) % HID] = np.where(np.arange(D) % 2 == 0, 1.0, -1.0)
    return wq, wp, wk


def _random_weights(seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((H * D, R)) / np.sqrt(R), rng.uniform(-1, 1, (H, HID)) / np.sqrt(HID),
            rng.standard_normal((D, HID)) / np.sqrt(HID))


def _inputs(T, dtype, seed):
    rng = np.random.default_rng(seed)
    hidden = _to_bits(rng.standard_normal((T, HID)), dtype)
    qc = _to_bits(rng.standard_normal((T, R)), dtype)
    c, s = _cos_sin(T, dtype, seed=seed)
    return hidden, qc, c, s


def _run_query_only(hidden, qc, c, s, wq, wp, dtype, scale, wp_dev=None):
    from nanovllm_amd.dsa_indexer_project import dsa_indexer_project_query_only

    T = hidden.shape[0]
    q_out = torch.empty(T, H, D, dtype=dtype, device="cuda")
    w_out = torch.empty(T, H, dtype=dtype, device="cuda")
    dsa_indexer_project_query_only(_dev(hidden, dtype), _dev(qc, dtype), _dev(c, dtype), _dev(s, dtype),
                                   _dev(wq, dtype), wp_dev if wp_dev is not None else _dev(wp, dtype), q_out, w_out,
                                   n_head=H, head_dim=D, rope_dim=ROPE, score_scale=scale)
    torch.cuda.synchronize()
    return bits(q_out), bits(w_out)


def _close(got, expect, dtype, min_exact=0.98, pairs=False):
    """Within two 16-bit steps of the value (of the pair's norm for rotated
    pairs: an input one step off moves both outputs by up to a step of the
    larger one), and mostly exact.  The values are O(1)."""
    g = O.bits_to_f32(got, dname(dtype)).astype(np.float64)
    e = O.bits_to_f32(expect, dname(dtype)).astype(np.float64)
    mag = np.abs(e)
    if pairs:
        mag = np.repeat(np.hypot(e[..., 0::2], e[..., 1::2]), 2, axis=-1)
    rel = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    # values near zero: the fp32 sums' own error (~1e-6 here) is the floor
    err = np.abs(g - e) - rel * np.maximum(mag, 2.0 ** -6)
    assert np.all(err <= 0), f"worst excess {float(err.max()):.3g}"
    exact = float(np.mean(got == expect))
    assert exact >= min_exact, exact


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,scale", [(1, 1.0), (24, 1.0), (64, 0.0883883), (65, 1.0), (130, 0.5)])
def test_project_query_only_one_hot_bit_exact(dtype, T, scale):
    print(f"PROJECT one-hot {dtype} T={T} scale={scale}", flush=True)
    hidden, qc, c, s = _inputs(T, dtype, seed=T)
    wq, wp, _ = _one_hot()
    wq16, wp16 = _to_bits(wq, dtype), _to_bits(wp, dtype)
    q, w = _run_query_only(hidden, qc, c, s, wq16, wp16, dtype, scale)
    eq, ew = I.project_query_only(hidden, qc, c, s, wq16, wp16, H, D, ROPE, scale, dname(dtype))
    assert np.array_equal(q, eq)
    assert np.array_equal(w, ew)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [3, 24, 64])
def test_project_query_only_random_close(dtype, T):
    print(f"PROJECT random {dtype} T={T}", flush=True)
    hidden, qc, c, s = _inputs(T, dtype, seed=100 + T)
    wq, wp, _ = _random_weights(T)
    wq16, wp16 = _to_bits(wq, dtype), _to_bits(wp, dtype)
    q, w = _run_query_only(hidden, qc, c, s, wq16, wp16, dtype, 1.0)
    eq, ew = I.project_query_only(hidden, qc, c, s, wq16, wp16, H, D, ROPE, 1.0, dname(dtype))
    _close(q[..., ROPE:], eq[..., ROPE:], dtype)
    _close(q[..., :ROPE], eq[..., :ROPE], dtype, min_exact=0.95, pairs=True)
    _close(w, ew, dtype)


def test_project_query_only_fp32_weights_proj():
    """weights_proj in fp32 (the reference's dtype-mismatch branch, :82-86)."""
    dtype = torch.bfloat16
    T = 24
    hidden, qc, c, s = _inputs(T, dtype, seed=7)
    wq, wp, _ = _random_weights(7)
    wq16 = _to_bits(wq, dtype)
    wp32 = np.asarray(wp, np.float32)
    q, w = _run_query_only(hidden, qc, c, s, wq16, None, dtype, 0.25,
                           wp_dev=torch.from_numpy(wp32).to("cuda"))
    eq, ew = I.project_query_only(hidden, qc, c, s, wq16, wp32, H, D, ROPE, 0.25, "bf16")
    _close(w, ew, dtype)
    _close(q[..., ROPE:], eq[..., ROPE:], dtype)
    _close(q[..., :ROPE], eq[..., :ROPE], dtype, min_exact=0.95, pairs=True)


def test_project_full_prefill():
    from nanovllm_amd.dsa_indexer_project import dsa_indexer_project

    dtype = torch.bfloat16
    T = 200
    print(f"PROJECT full T={T}", flush=True)
    hidden, qc, c, s = _inputs(T, dtype, seed=9)
    wq, wp, wk = _one_hot()
    kw = _to_bits(np.linspace(0.75, 1.25, D), dtype)
    kb = _to_bits(np.linspace(-0.125, 0.125, D), dtype)
    q_out = torch.empty(T, H, D, dtype=dtype, device="cuda")
    k_out = torch.empty(T, D, dtype=dtype, device="cuda")
    w_out = torch.empty(T, H, dtype=dtype, device="cuda")
    dsa_indexer_project(_dev(hidden, dtype), _dev(qc, dtype), _dev(c, dtype), _dev(s, dtype),
                        _dev(_to_bits(wq, dtype), dtype), _dev(_to_bits(wk, dtype), dtype), _dev(kw, dtype),
                        _dev(kb, dtype), torch.from_numpy(wp).to("cuda"), q_out, k_out, w_out, n_head=H,
                        head_dim=D, rope_dim=ROPE, score_scale=1.0)
    torch.cuda.synchronize()
    eq, ek, ew = I.project_full(hidden, qc, c, s, _to_bits(wq, dtype), _to_bits(wk, dtype), kw, kb, wp, H, D, ROPE,
                                1.0)
    assert np.array_equal(bits(q_out), eq)
    assert np.array_equal(bits(w_out), ew)
    torch.testing.assert_close(k_out.float().cpu(), torch.from_numpy(O.bits_to_f32(ek)), atol=0.05, rtol=0.025)


def test_project_errors():
    from nanovllm_amd.dsa_indexer_project import dsa_indexer_project, dsa_indexer_project_query_only

    dtype = torch.bfloat16
    T = 2
    hidden = torch.zeros(T, HID, dtype=dtype, device="cuda")
    qc = torch.zeros(T, R, dtype=dtype, device="cuda")
    cos = torch.zeros(T, 1, 1, ROPE, dtype=dtype, device="cuda")
    wq = torch.zeros(H * D, R, dtype=dtype, device="cuda")
    wp = torch.zeros(H, HID, dtype=dtype, device="cuda")
    with pytest.raises(ValueError, match=r"q_index_out shape must be \(2, 32, 128\)"):
        dsa_indexer_project_query_only(hidden, qc, cos, cos, wq, wp, torch.empty(T, H, 64, dtype=dtype, device="cuda"),
                                       torch.empty(T, H, dtype=dtype, device="cuda"), n_head=H, head_dim=D,
                                       rope_dim=ROPE, score_scale=1.0)
    with pytest.raises(ValueError, match=r"index_weights_out shape must be \(2, 32\)"):
        dsa_indexer_project_query_only(hidden, qc, cos, cos, wq, wp, torch.empty(T, H, D, dtype=dtype, device="cuda"),
                                       torch.empty(T, 16, dtype=dtype, device="cuda"), n_head=H, head_dim=D,
                                       rope_dim=ROPE, score_scale=1.0)
    with pytest.raises(ValueError, match="index_k_out must use dtype"):
        dsa_indexer_project(hidden, qc, cos, cos, wq, torch.zeros(D, HID, dtype=dtype, device="cuda"),
                            torch.ones(D, dtype=dtype, device="cuda"), None, wp.float(),
                            torch.empty(T, H, D, dtype=dtype, device="cuda"),
                            torch.empty(T, D, dtype=torch.float16, device="cuda"),
                            torch.empty(T, H, dtype=dtype, device="cuda"), n_head=H, head_dim=D, rope_dim=ROPE,
                            score_scale=1.0)
    with pytest.raises(RuntimeError, match="multiple of 256"):
        dsa_indexer_project_query_only(hidden, qc[:, :2000].contiguous(), cos, cos, wq[:, :2000].contiguous(), wp,
                                       torch.empty(T, H, D, dtype=dtype, device="cuda"),
                                       torch.empty(T, H, dtype=dtype, device="cuda"), n_head=H, head_dim=D,
                                       rope_dim=ROPE, score_scale=1.0)
