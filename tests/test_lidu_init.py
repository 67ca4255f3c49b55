"""First-decode LIDU initialisation: initialize_lidu_row(_shared)
(reference nanovllm/models/dsa_offload_ops.py:251-411).

CPU: the oracle against what the mathematics fixes -- the closed-form index
(score == token id, ut_ops/test_fused_li_manage.py:146-173), the linear score
computed a second way (one effective query, no ReLU), tie order, the
reference's argument errors and the shared layer's copy.
GPU: initialize_lidu_row(_shared) bit-exact against the oracle (pool row,
HBM rows) on margin-guarded random inputs and on the closed form.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits, ints
from oracle import dsa_oracle as O

TOPK = O.TOPK


def _digit_keys(n_blocks: int) -> np.ndarray:
    ids = np.arange(n_blocks * 128)
    k = np.zeros((n_blocks, 128, 1, 128), np.float32)
    flat = k.reshape(-1, 128)
    flat[:, 0] = ids % 64
    flat[:, 1] = (ids // 64) % 64
    flat[:, 2] = (ids // 4096) % 64
    flat[:, 3] = ids // 262144
    return k


def _digit_query(heads: int):
    q = np.zeros((heads, 128), np.float32)
    q[0, :4] = [1, 64, 4096, 262144]
    w = np.zeros(heads, np.float32)
    w[0] = 1
    return q, w


def _caches(rng, blocks: int):
    dkpe = rng.integers(0, 1 << 16, (blocks, 128, 64), dtype=np.uint16)
    dckv = rng.integers(0, 1 << 16, (blocks, 128, 512), dtype=np.uint16)
    return dkpe, dckv


def test_linear_scores_are_one_effective_query_without_relu():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((32, 128))
    w = rng.uniform(-1, 1, 32)
    k = rng.standard_normal((50, 128))
    s = O.linear_index_scores(q, w, k)
    q_eff = w @ q  # sum_h w_h q_h: the score is linear in the key
    assert np.allclose(s, k @ q_eff, rtol=1e-12, atol=1e-9)
    # the LIM score (with ReLU) differs on these inputs: negative dot products occur
    assert not np.allclose(s, O.index_scores(q, w, k))


def test_lidu_init_closed_form_last_tokens():
    rng = np.random.default_rng(3)
    n_blocks, c = 40, 3000  # 5120 tokens
    n = n_blocks * 128
    keys = O.f32_to_bits(_digit_keys(n_blocks))
    q, w = _digit_query(32)
    table = rng.permutation(n_blocks).astype(np.int32)
    inv = np.empty_like(table)
    inv[table] = np.arange(n_blocks)
    # key rows are stored through the table: logical block j lives at physical table[j]
    keys_phys = keys[inv]
    dkpe, dckv = _caches(rng, n_blocks)
    h_blocks = (c + 127) // 128
    hkpe = np.zeros((h_blocks, 128, 64), np.uint16)
    hckv = np.zeros((h_blocks, 128, 512), np.uint16)
    htab = rng.permutation(h_blocks).astype(np.int32)
    slots = np.full(n, 123, np.int32)
    src, dst = O.initialize_lidu_row(O.f32_to_bits(q), O.f32_to_bits(w), keys_phys, table, n, c, slots, hkpe, hckv,
                                     dkpe, dckv, htab, table)
    assert np.array_equal(src, np.arange(n - c, n))
    assert np.array_equal(dst, np.arange(c))
    expect = np.full(n, -1, np.int32)
    expect[n - c:] = np.arange(c)
    assert np.array_equal(slots, expect)
    for i in (0, 1, 777, c - 1):  # slot i holds token n - c + i
        t = n - c + i
        d = htab[i // 128] * 128 + i % 128
        sr = table[t // 128] * 128 + t % 128
        assert np.array_equal(hckv.reshape(-1, 512)[d], dckv.reshape(-1, 512)[sr])
        assert np.array_equal(hkpe.reshape(-1, 64)[d], dkpe.reshape(-1, 64)[sr])


def test_lidu_init_ties_take_lowest_tokens():
    rng = np.random.default_rng(5)
    n_blocks, c = 24, 2048
    n = n_blocks * 128
    keys = np.zeros((n_blocks, 128, 1, 128), np.uint16)  # every score is 0
    q = O.f32_to_bits(rng.standard_normal((32, 128)).astype(np.float32))
    w = O.f32_to_bits(rng.uniform(0, 1, 32).astype(np.float32))
    table = np.arange(n_blocks, dtype=np.int32)
    dkpe, dckv = _caches(rng, n_blocks)
    hkpe = np.zeros((16, 128, 64), np.uint16)
    hckv = np.zeros((16, 128, 512), np.uint16)
    slots = np.zeros(n, np.int32)
    src, _ = O.initialize_lidu_row(q, w, keys, table, n, c, slots, hkpe, hckv, dkpe, dckv, np.arange(16), table)
    assert np.array_equal(src, np.arange(c))
    assert (slots[c:] == -1).all()


def test_lidu_init_argument_errors_and_noop():
    args = dict(query=None, weights=None, key_cache=None, index_table_row=None, slots_row=None, hbm_kpe=None,
                hbm_ckv=None, dram_kpe=None, dram_ckv=None, hbm_table_row=None, dram_table_row=None)
    assert O.initialize_lidu_row(candidate_len=4096, cache_tokens=0, **args) is None
    with pytest.raises(ValueError, match="must be >= 2048, got 2047"):
        O.initialize_lidu_row(candidate_len=4096, cache_tokens=2047, **args)
    with pytest.raises(ValueError, match="cache budget 4096 exceeds source length 3968"):
        O.initialize_lidu_row(candidate_len=3968, cache_tokens=4096, **args)
    with pytest.raises(ValueError, match="complete blocks"):
        O.initialize_lidu_row(candidate_len=4100, cache_tokens=2048, **args)


def test_lidu_shared_copies_owner_mapping_and_checks_count():
    rng = np.random.default_rng(9)
    n, c = 4096, 2100
    slots = np.full(n, -1, np.int32)
    toks = np.sort(rng.choice(n, c, replace=False))
    slots[toks] = rng.permutation(c)
    dkpe, dckv = _caches(rng, 32)
    hkpe = np.zeros((17, 128, 64), np.uint16)
    hckv = np.zeros((17, 128, 512), np.uint16)
    htab = rng.permutation(17).astype(np.int32)
    dtab = rng.permutation(32).astype(np.int32)
    src, dst = O.initialize_lidu_row_shared(slots, c, hkpe, hckv, dkpe, dckv, htab, dtab)
    assert np.array_equal(src, toks) and np.array_equal(dst, slots[toks])
    t = int(toks[17])
    d = int(slots[t])
    assert np.array_equal(hckv.reshape(-1, 512)[htab[d // 128] * 128 + d % 128],
                          dckv.reshape(-1, 512)[dtab[t // 128] * 128 + t % 128])
    assert O.initialize_lidu_row_shared(slots, 0, hkpe, hckv, dkpe, dckv, htab, dtab) is None
    with pytest.raises(RuntimeError, match="found 2100 cached tokens, expected 2101"):
        O.initialize_lidu_row_shared(slots, c + 1, hkpe, hckv, dkpe, dckv, htab, dtab)


# --------------------------------------------------------------------------
# GPU
def _guard_linear(keys_bits, table, n, q_bits, w_bits, c, max_iter=64):
    """Margin guard at the top-C boundary of the linear score: while the
    boundary gap is below both tokens' fp32 error bounds, scale the inside
    token's key row by 2 (positive score) or 1/2 (negative): exact in bf16,
    it moves that score up and leaves every other score unchanged."""
    q = O.bits_to_f32(q_bits).astype(np.float64).reshape(-1, 128)
    w = O.bits_to_f32(w_bits).astype(np.float64).reshape(-1)
    rows = keys_bits.reshape(-1, 128)
    phys = table[np.arange(n) // 128].astype(np.int64) * 128 + np.arange(n) % 128
    for _ in range(max_iter):
        k = O.bits_to_f32(rows[phys]).astype(np.float64)
        s = (k @ q.T) @ w
        err = 2.0 ** -24 * 256 * (np.abs(k) @ np.abs(q).T) @ np.abs(w)
        order = np.lexsort((np.arange(n), -s))
        t_in, t_out = order[c - 1], order[c]
        if s[t_in] - s[t_out] > err[t_in] + err[t_out]:
            return
        f = O.bits_to_f32(rows[phys[t_in]]) * (2.0 if s[t_in] > 0 else 0.5)
        rows[phys[t_in]] = O.f32_to_bits(f.astype(np.float32))
    raise AssertionError("margin guard did not converge")


def _init_case(seed, n_blocks, c, heads=32, dtype="bf16", closed_form=False):
    rng = np.random.default_rng(seed)
    n = n_blocks * 128
    table = rng.permutation(n_blocks + 3)[:n_blocks].astype(np.int32)
    if closed_form:
        keys = np.zeros((n_blocks + 3, 128, 1, 128), np.uint16)
        logical = O.f32_to_bits(_digit_keys(n_blocks), dtype)
        keys[table] = logical
        q, w = _digit_query(heads)
        if dtype == "f16":
            q[0, 3] = 0.0  # 262144 overflows fp16; every id here is < 262144
        qb, wb = O.f32_to_bits(q, dtype), O.f32_to_bits(w, dtype)
    else:
        keys = O.f32_to_bits(rng.standard_normal((n_blocks + 3, 128, 1, 128)).astype(np.float32), dtype)
        qb = O.f32_to_bits(rng.standard_normal((heads, 128)).astype(np.float32), dtype)
        wb = O.f32_to_bits(rng.uniform(-0.2, 1, heads).astype(np.float32), dtype)
        if dtype == "bf16":
            _guard_linear(keys, table, n, qb, wb, c)
    d_blocks = n_blocks + 2
    dkpe, dckv = _caches(rng, d_blocks)
    dtab = rng.permutation(d_blocks)[:n_blocks].astype(np.int32)
    h_blocks = (c + 127) // 128 + 2
    hkpe = rng.integers(0, 1 << 16, (h_blocks, 128, 64), dtype=np.uint16)
    hckv = rng.integers(0, 1 << 16, (h_blocks, 128, 512), dtype=np.uint16)
    htab = rng.permutation(h_blocks).astype(np.int32)[: (c + 127) // 128 + 1]
    cap = (n_blocks + 1) * 128
    slots = rng.integers(-1, c, cap).astype(np.int32)  # stale contents: overwritten entirely
    return dict(q=qb, w=wb, keys=keys, table=np.concatenate([table, [-1]]).astype(np.int32), n=n, c=c, slots=slots,
                hkpe=hkpe, hckv=hckv, dkpe=dkpe, dckv=dckv, htab=htab, dtab=np.concatenate([dtab, [-1]]).astype(np.int32),
                dtype=dtype)


def _to_gpu(case):
    import nanovllm_amd.host_memory as hm

    tdt = torch.bfloat16 if case["dtype"] == "bf16" else torch.float16
    f16 = lambda a: torch.from_numpy(a.view(np.int16)).view(tdt).cuda()  # noqa: E731
    i32 = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    g = dict(query=f16(case["q"]), weights=f16(case["w"]), index_cache=f16(case["keys"]),
             index_block_table=i32(case["table"]), cache_slots_row=i32(case["slots"]), hbm_kpe=f16(case["hkpe"]),
             hbm_ckv=f16(case["hckv"]), hbm_block_table=i32(case["htab"]), dram_block_table=i32(case["dtab"]))
    for name, arr in (("dram_kpe", case["dkpe"]), ("dram_ckv", case["dckv"])):
        gpu, host = hm.host_mapped_pair(arr.shape, tdt)
        host.copy_(torch.from_numpy(arr.view(np.int16)).view(tdt))
        g[name] = gpu
    return g


def _oracle_init(case):
    slots, hkpe, hckv = case["slots"].copy(), case["hkpe"].copy(), case["hckv"].copy()
    O.initialize_lidu_row(case["q"], case["w"], case["keys"], case["table"], case["n"], case["c"], slots, hkpe, hckv,
                          case["dkpe"], case["dckv"], case["htab"], case["dtab"], dtype=case["dtype"])
    return slots, hkpe, hckv


@pytest.mark.gpu
@pytest.mark.parametrize("seed,n_blocks,c,heads,dtype,closed", [
    (1, 40, 3000, 32, "bf16", True),
    (2, 48, 2048, 32, "bf16", False),
    (3, 72, 5000, 64, "bf16", False),
    (4, 24, 2048, 32, "f16", True),
    (5, 256, 2048, 32, "bf16", False),   # 32768 tokens: the largest source whose keys stay in registers
    (6, 320, 8192, 32, "bf16", True),    # 40960 tokens: the streaming kernel
    (7, 530, 3000, 32, "bf16", False),   # 67840 tokens: the streaming kernel
])
def test_gpu_initialize_lidu_row_matches_oracle(seed, n_blocks, c, heads, dtype, closed):
    from nanovllm_amd import dsa_offload_ops as ops

    case = _init_case(seed, n_blocks, c, heads, dtype, closed)
    print(f"LIDU-INIT seed={seed} n={case['n']} c={c} heads={heads} {dtype} closed={closed}", flush=True)
    slots, hkpe, hckv = _oracle_init(case)
    g = _to_gpu(case)
    out = ops.initialize_lidu_row(candidate_len=case["n"], cache_tokens=c, block_size=128, **g)
    torch.cuda.synchronize()
    assert out[0] is g["hbm_kpe"] and out[1] is g["hbm_ckv"]
    assert np.array_equal(ints(g["cache_slots_row"]), slots)
    assert np.array_equal(bits(g["hbm_ckv"]), hckv)
    assert np.array_equal(bits(g["hbm_kpe"]), hkpe)


def _unaligned(t: torch.Tensor) -> torch.Tensor:
    """A copy of 1-D ``t`` whose data starts 4 bytes into an allocation (not
    16-byte aligned), so the kernels take their element-wise path."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    view = buf[1:]
    view.copy_(t)
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.gpu
def test_gpu_initialize_lidu_row_unaligned_pool_row():
    """32768 candidates (keys in registers) written into a pool row that is
    not 16-byte aligned."""
    from nanovllm_amd import dsa_offload_ops as ops

    case = _init_case(5, 256, 2048, 32, "bf16", False)
    print(f"LIDU-INIT unaligned row n={case['n']}", flush=True)
    slots, hkpe, hckv = _oracle_init(case)
    g = _to_gpu(case)
    g["cache_slots_row"] = _unaligned(g["cache_slots_row"])
    ops.initialize_lidu_row(candidate_len=case["n"], cache_tokens=2048, block_size=128, **g)
    torch.cuda.synchronize()
    assert np.array_equal(ints(g["cache_slots_row"]), slots)
    assert np.array_equal(bits(g["hbm_ckv"]), hckv)
    assert np.array_equal(bits(g["hbm_kpe"]), hkpe)


@pytest.mark.gpu
@pytest.mark.parametrize("aligned", [True, False])
def test_gpu_initialize_lidu_row_shared_long_row(aligned):
    """An owner pool row of 67840 entries (groups of 8 x 4096 entries, the
    last one partial) with 5000 cached tokens spread over it, 16-byte
    aligned or not: the shared layer copies exactly the owner's mapping."""
    from nanovllm_amd import dsa_offload_ops as ops

    c = 5000
    case = _init_case(12, 530, c, closed_form=True)
    rng = np.random.default_rng(13)
    slots = np.full(case["slots"].shape, -1, np.int32)
    slots[rng.choice(case["n"], c, replace=False)] = rng.permutation(c).astype(np.int32)
    hkpe, hckv = case["hkpe"].copy(), case["hckv"].copy()
    O.initialize_lidu_row_shared(slots, c, hkpe, hckv, case["dkpe"], case["dckv"], case["htab"], case["dtab"])
    print(f"LIDU-SHARED row {slots.shape[0]} entries, {c} cached, aligned={aligned}", flush=True)
    g = _to_gpu(dict(case, slots=slots))
    row = g["cache_slots_row"] if aligned else _unaligned(g["cache_slots_row"])
    ops.initialize_lidu_row_shared(cache_slots_row=row, cache_tokens=c, hbm_kpe=g["hbm_kpe"], hbm_ckv=g["hbm_ckv"],
                                   dram_kpe=g["dram_kpe"], dram_ckv=g["dram_ckv"],
                                   hbm_block_table=g["hbm_block_table"], dram_block_table=g["dram_block_table"])
    torch.cuda.synchronize()
    assert np.array_equal(ints(row), slots)  # the owner's row is read, not written
    assert np.array_equal(bits(g["hbm_ckv"]), hckv)
    assert np.array_equal(bits(g["hbm_kpe"]), hkpe)


@pytest.mark.gpu
@pytest.mark.parametrize("n_blocks", [200, 300])
def test_gpu_initialize_lidu_row_all_ties(n_blocks):
    """Every index key zero: every score is 0, so the C selected tokens are the
    C lowest (ties at the threshold go to the lower tokens) and slot i goes
    to token i; 25600 tokens (keys in registers, the last register chunk cut
    at n) and 38400 (the streaming kernel)."""
    from nanovllm_amd import dsa_offload_ops as ops

    c = 2048
    case = _init_case(11, n_blocks, c, 32, "bf16", closed_form=True)
    case["keys"][:] = 0
    print(f"LIDU-INIT all ties n={case['n']} c={c}", flush=True)
    slots, hkpe, hckv = _oracle_init(case)
    expect = np.full(case["slots"].shape, -1, np.int32)
    expect[:c] = np.arange(c, dtype=np.int32)
    assert np.array_equal(slots, expect)
    g = _to_gpu(case)
    ops.initialize_lidu_row(candidate_len=case["n"], cache_tokens=c, block_size=128, **g)
    torch.cuda.synchronize()
    assert np.array_equal(ints(g["cache_slots_row"]), slots)
    assert np.array_equal(bits(g["hbm_ckv"]), hckv)
    assert np.array_equal(bits(g["hbm_kpe"]), hkpe)


@pytest.mark.gpu
def test_gpu_initialize_lidu_row_shared_and_errors():
    from nanovllm_amd import dsa_offload_ops as ops

    case = _init_case(7, 32, 2500)
    slots, _, _ = _oracle_init(case)  # the owner's pool row
    rng = np.random.default_rng(8)
    other = dict(case, dkpe=_caches(rng, 34)[0], dckv=_caches(rng, 34)[1], slots=slots)
    hkpe, hckv = other["hkpe"].copy(), other["hckv"].copy()
    O.initialize_lidu_row_shared(slots, 2500, hkpe, hckv, other["dkpe"], other["dckv"], other["htab"], other["dtab"])
    g = _to_gpu(other)
    ops.initialize_lidu_row_shared(cache_slots_row=g["cache_slots_row"], cache_tokens=2500, hbm_kpe=g["hbm_kpe"],
                                   hbm_ckv=g["hbm_ckv"], dram_kpe=g["dram_kpe"], dram_ckv=g["dram_ckv"],
                                   hbm_block_table=g["hbm_block_table"], dram_block_table=g["dram_block_table"])
    torch.cuda.synchronize()
    assert np.array_equal(bits(g["hbm_ckv"]), hckv) and np.array_equal(bits(g["hbm_kpe"]), hkpe)
    with pytest.raises(RuntimeError, match="found 2500 cached tokens, expected 2501"):
        ops.initialize_lidu_row_shared(cache_slots_row=g["cache_slots_row"], cache_tokens=2501, hbm_kpe=g["hbm_kpe"],
                                       hbm_ckv=g["hbm_ckv"], dram_kpe=g["dram_kpe"], dram_ckv=g["dram_ckv"],
                                       hbm_block_table=g["hbm_block_table"],
                                       dram_block_table=g["dram_block_table"])
    # the reference's argument errors, raised before any launch; C <= 0 is a no-op
    base = dict(query=g["query"], weights=g["weights"], index_cache=g["index_cache"],
                index_block_table=g["index_block_table"], cache_slots_row=g["cache_slots_row"], hbm_kpe=g["hbm_kpe"],
                hbm_ckv=g["hbm_ckv"], dram_kpe=g["dram_kpe"], dram_ckv=g["dram_ckv"],
                hbm_block_table=g["hbm_block_table"], dram_block_table=g["dram_block_table"], block_size=128)
    before = ints(g["cache_slots_row"])
    ops.initialize_lidu_row(candidate_len=4096, cache_tokens=0, **base)
    with pytest.raises(ValueError, match="got 100"):
        ops.initialize_lidu_row(candidate_len=4096, cache_tokens=100, **base)
    with pytest.raises(ValueError, match="exceeds source length"):
        ops.initialize_lidu_row(candidate_len=2048, cache_tokens=2176, **base)
    with pytest.raises(ValueError, match="complete blocks"):
        ops.initialize_lidu_row(candidate_len=4000, cache_tokens=2048, **base)
    torch.cuda.synchronize()
    assert np.array_equal(ints(g["cache_slots_row"]), before)
