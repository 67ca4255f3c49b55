"""Pins of the indexer-projection oracle (oracle/indexer_oracle.py), CPU only.

* RoPE: identity (cos 1, sin 0) and quarter turn (cos 0, sin 1 gives
  (-odd, even)) exactly; a literal pure-Python restatement of the AscendC
  steps (uint32 pair swap by shifts, [-1, +1] sign pair, fp32 Mul/Mul/Add,
  dsa_indexer_project_kernel.cpp:118-163) on a small case; a float64 textbook
  rotation within one 16-bit ulp; rotating by theta then -theta.
* Projections: the reference test's one-hot weights
  (ut_ops/test_glm_dsa_indexer.py:127-192) give closed forms for q, k and the
  weights (q_c[:, source] * sign, ...); k's layer norm against torch's
  float64 layer_norm.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O
from oracle import indexer_oracle as I

H, D, R, HID, ROPE = 32, 128, 2048, 6144, 64


def _bits(x, dtype="bf16"):
    return O.f32_to_bits(np.asarray(x, np.float32), dtype).reshape(np.shape(x))


def _angles(T, rope=ROPE, seed=0):
    rng = np.random.default_rng(seed)
    pos = rng.integers(1, 40000, size=(T, 1)).astype(np.float64)
    freq = 10000.0 ** (-np.arange(rope // 2) * 2.0 / rope)
    ang = np.repeat(pos * freq[None, :], 2, axis=1)
    return np.cos(ang), np.sin(ang)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_rope_identity_and_quarter_turn(dtype):
    rng = np.random.default_rng(1)
    T = 3
    q = _bits(rng.standard_normal((T, 4, D)), dtype)
    ones, zeros = _bits(np.ones((T, ROPE)), dtype), _bits(np.zeros((T, ROPE)), dtype)
    a = q.copy()
    I.query_rope_inplace(a, ones, zeros, ROPE, dtype)
    assert np.array_equal(a, q)
    b = q.copy()
    I.query_rope_inplace(b, zeros, ones, ROPE, dtype)
    x = O.bits_to_f32(q, dtype)
    expect = x.copy()
    expect[..., 0:ROPE:2] = -x[..., 1:ROPE:2]
    expect[..., 1:ROPE:2] = x[..., 0:ROPE:2]
    assert np.array_equal(b, _bits(expect, dtype))
    assert np.array_equal(b[..., ROPE:], q[..., ROPE:])  # dims past rope_dim untouched


def _f32(v):
    return struct.unpack("<f", struct.pack("<f", v))[0]


def test_rope_literal_ascend_steps_small():
    """Per pair: pack (even, odd) as one uint32 (little endian: even low),
    swap halves with shifts and OR, multiply by the [-1, +1] sign pair, then
    fp32 Mul, Mul, Add and a round to nearest even -- scalar by scalar."""
    rng = np.random.default_rng(2)
    T, nh = 2, 3
    q = _bits(rng.standard_normal((T, nh, 32)))
    c = _bits(rng.uniform(-1, 1, (T, 16)))
    s = _bits(rng.uniform(-1, 1, (T, 16)))
    got = q.copy()
    I.query_rope_inplace(got, c, s, 16)
    sign = struct.unpack("<HH", struct.pack("<I", 0x3F80BF80))  # (low, high) = (-1, +1) in bf16
    sign_f = [O.bits_to_f32(np.array([v], np.uint16))[0] for v in sign]
    for t in range(T):
        for h in range(nh):
            for i in range(8):
                lo, hi = int(q[t, h, 2 * i]), int(q[t, h, 2 * i + 1])
                packed = lo | (hi << 16)
                swapped = ((packed << 16) | (packed >> 16)) & 0xFFFFFFFF
                sw = [swapped & 0xFFFF, swapped >> 16]
                for j in range(2):
                    x = float(O.bits_to_f32(np.array([(lo, hi)[j]], np.uint16))[0])
                    rot = _f32(float(O.bits_to_f32(np.array([sw[j]], np.uint16))[0]) * sign_f[j])
                    cv = float(O.bits_to_f32(np.array([c[t, 2 * i + j]], np.uint16))[0])
                    sv = float(O.bits_to_f32(np.array([s[t, 2 * i + j]], np.uint16))[0])
                    out = _f32(_f32(x * cv) + _f32(rot * sv))
                    assert got[t, h, 2 * i + j] == _bits(np.array([out]))[0], (t, h, i, j)
            assert np.array_equal(got[t, h, 16:], q[t, h, 16:])


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_rope_matches_float64_rotation(dtype):
    rng = np.random.default_rng(3)
    T = 8
    q = _bits(rng.standard_normal((T, H, D)), dtype)
    cos64, sin64 = _angles(T)
    c, s = _bits(cos64, dtype), _bits(sin64, dtype)
    got = q.copy()
    I.query_rope_inplace(got, c, s, ROPE, dtype)
    x = O.bits_to_f32(q, dtype).astype(np.float64)[..., :ROPE]
    cf = O.bits_to_f32(c, dtype).astype(np.float64)[:, None, :]
    sf = O.bits_to_f32(s, dtype).astype(np.float64)[:, None, :]
    e, o = x[..., 0::2], x[..., 1::2]
    ref = np.empty_like(x)
    ref[..., 0::2] = e * cf[..., 0::2] - o * sf[..., 0::2]
    ref[..., 1::2] = o * cf[..., 1::2] + e * sf[..., 1::2]
    g = O.bits_to_f32(got[..., :ROPE], dtype).astype(np.float64)
    ulp = 2.0 ** (-8 if dtype == "bf16" else -11)
    assert np.all(np.abs(g - ref) <= ulp * np.maximum(np.abs(ref), 2.0 ** -14) + 1e-30)
    # and rotating back by -theta restores x
    back = got.copy()
    I.query_rope_inplace(back, c, _bits(-O.bits_to_f32(s, dtype), dtype), ROPE, dtype)
    xb = O.bits_to_f32(back[..., :ROPE], dtype).astype(np.float64)
    # cos^2 + sin^2 is 1 only to within the 16-bit rounding of cos and sin,
    # so the error scales with the pair's norm
    norm = np.repeat(np.hypot(x[..., 0::2], x[..., 1::2]), 2, axis=-1)
    assert np.all(np.abs(xb - x) <= 4 * ulp * np.maximum(norm, 2.0 ** -8))


def _one_hot(dtype="bf16"):
    """The reference test's structured projections (test_glm_dsa_indexer.py:127-192)."""
    q_rows = H * D
    q_source = (np.arange(q_rows) * 17 + 11) % R
    q_sign = np.where(np.arange(q_rows) % 3 == 0, -1.0, 1.0)
    wq = np.zeros((q_rows, R), np.float32)
    wq[np.arange(q_rows), q_source] = q_sign
    k_source = (np.arange(D) * 29 + 7) % HID
    k_sign = np.where(np.arange(D) % 2 == 0, 1.0, -1.0)
    wk = np.zeros((D, HID), np.float32)
    wk[np.arange(D), k_source] = k_sign
    w_source = (np.arange(H) * 43 + 5) % HID
    w_sign = np.where(np.arange(H) % 2 == 0, 1.0, -1.0)
    wp = np.zeros((H, HID), np.float32)
    wp[np.arange(H), w_source] = w_sign
    return wq, q_source, q_sign, wk, k_source, k_sign, wp, w_source, w_sign


@pytest.mark.parametrize("scale", [1.0, 0.0883883])
def test_project_query_only_one_hot_closed_form(scale):
    rng = np.random.default_rng(4)
    T = 3
    hidden = _bits(rng.standard_normal((T, HID)))
    qc = _bits(rng.standard_normal((T, R)))
    cos64, sin64 = _angles(T)
    c, s = _bits(cos64), _bits(sin64)
    wq, q_source, q_sign, _, _, _, wp, w_source, w_sign = _one_hot()
    q, w = I.project_query_only(hidden, qc, c, s, _bits(wq), _bits(wp), H, D, ROPE, scale)
    proj = (O.bits_to_f32(qc)[:, q_source] * q_sign).reshape(T, H, D)
    assert np.array_equal(q[..., ROPE:], _bits(proj[..., ROPE:]))  # the projection is exact
    x = proj[..., :ROPE].astype(np.float64)
    cf, sf = O.bits_to_f32(c).astype(np.float64)[:, None, :], O.bits_to_f32(s).astype(np.float64)[:, None, :]
    ref = np.empty_like(x)
    ref[..., 0::2] = x[..., 0::2] * cf[..., 0::2] - x[..., 1::2] * sf[..., 0::2]
    ref[..., 1::2] = x[..., 1::2] * cf[..., 1::2] + x[..., 0::2] * sf[..., 1::2]
    g = O.bits_to_f32(q[..., :ROPE]).astype(np.float64)
    assert np.all(np.abs(g - ref) <= 2.0 ** -8 * np.maximum(np.abs(ref), 2.0 ** -14))
    wexp = O.bits_to_f32(hidden)[:, w_source] * w_sign
    if scale != 1.0:
        wexp = np.float32(wexp) * np.float32(scale)  # the 16-bit product rounded again
    assert np.array_equal(w, _bits(wexp))
    # fp32 weights_proj: one rounding after the fp32 scale
    _, w32 = I.project_query_only(hidden, qc, c, s, _bits(wq), wp, H, D, ROPE, scale)
    assert np.array_equal(w32, _bits(np.float32(O.bits_to_f32(hidden)[:, w_source] * w_sign) * np.float32(scale)))


def test_project_full_k_layer_norm_against_torch():
    rng = np.random.default_rng(5)
    T = 4
    hidden = _bits(rng.standard_normal((T, HID)))
    qc = _bits(rng.standard_normal((T, R)))
    cos64, sin64 = _angles(T)
    c, s = _bits(cos64), _bits(sin64)
    wq, _, _, wk, k_source, k_sign, wp, w_source, w_sign = _one_hot()
    kw = _bits(np.linspace(0.75, 1.25, D))
    kb = _bits(np.linspace(-0.125, 0.125, D))
    q, k, w = I.project_full(hidden, qc, c, s, _bits(wq), _bits(wk), kw, kb, wp, H, D, ROPE, 1.0)
    kproj = O.bits_to_f32(hidden)[:, k_source] * k_sign  # exact
    ln = torch.nn.functional.layer_norm(torch.from_numpy(kproj.astype(np.float64)), (D,),
                                        torch.from_numpy(O.bits_to_f32(kw).astype(np.float64)),
                                        torch.from_numpy(O.bits_to_f32(kb).astype(np.float64)), eps=1e-6).numpy()
    kn = O.bits_to_f32(k[:, ROPE:]).astype(np.float64)
    assert np.all(np.abs(kn - ln[:, ROPE:]) <= 2.0 ** -8 * np.maximum(np.abs(ln[:, ROPE:]), 2.0 ** -14))
    assert np.array_equal(w, _bits(O.bits_to_f32(hidden)[:, w_source] * w_sign))
    q2, _ = I.project_query_only(hidden, qc, c, s, _bits(wq), _bits(wp), H, D, ROPE, 1.0)
    assert np.array_equal(q, q2)
