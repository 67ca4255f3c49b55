"""The C ABI library loads, exports every symbol include/nvdsa.h declares, and
rejects bad arguments on the host (no GPU needed: validation precedes any
HIP call).  Also checks the torch.library registration of the reference's
schemas."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "nvdsa.h"


def test_library_exports_every_header_symbol():
    from nanovllm_amd import _lib

    declared = _lib.exported_symbols_from_header(HEADER)
    assert len(declared) == 26, declared
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for name in declared:
        assert hasattr(_lib.lib, name)
    assert set(_lib.SIGNATURES) == set(declared)
    assert _lib.version().startswith("nvdsa")


def _desc(shape, dtype_code, device=0, contiguous=1, data=0x1000):
    from nanovllm_amd._lib import NvdsaTensor

    d = NvdsaTensor()
    d.data = data
    d.dtype = dtype_code
    d.ndim = len(shape)
    for i, s in enumerate(shape):
        d.shape[i] = s
    d.contiguous = contiguous
    d.device = device
    return d


def _scatter_descs(B=2, cap=16, blocks=4):
    from nanovllm_amd._lib import BFLOAT16, INT32

    return [
        _desc((B, cap), INT32), _desc((B, cap), INT32), _desc((B,), INT32), _desc((B, 2), INT32),
        _desc((B, 2), INT32), _desc((blocks, 128, 64), BFLOAT16), _desc((blocks, 128, 512), BFLOAT16),
        _desc((blocks, 128, 64), BFLOAT16, device=-1), _desc((blocks, 128, 512), BFLOAT16, device=-1),
    ]


@pytest.mark.parametrize("mutate,code,msg", [
    (lambda d: setattr(d[6], "ndim", 4), 1, "HBM CKV"),
    (lambda d: d[6].shape.__setitem__(2, 256), 1, "HBM CKV"),
    (lambda d: d[1].shape.__setitem__(1, 8), 1, "source and destination"),
    (lambda d: (d[0].shape.__setitem__(1, 70000), d[1].shape.__setitem__(1, 70000)), 1, "65536"),
    (lambda d: setattr(d[0], "dtype", 3), 2, "int32"),
    (lambda d: setattr(d[5], "dtype", 3), 2, "fp16 or bf16"),
    (lambda d: setattr(d[8], "dtype", 1), 2, "same dtype"),
    (lambda d: setattr(d[4], "contiguous", 0), 3, "contiguous"),
    (lambda d: setattr(d[3], "device", 1), 4, "same device"),
    (lambda d: setattr(d[5], "device", -1), 4, "same device"),  # HBM cache may not be host memory
    (lambda d: setattr(d[6], "data", 0x1008), 3, "aligned"),
])
def test_scatter_copy_validation(mutate, code, msg):
    from nanovllm_amd import _lib

    d = _scatter_descs()
    mutate(d)
    status = _lib.lib.nvdsa_scatter_copy(*[ctypes.byref(x) for x in d], None)
    assert status == code
    assert msg in _lib.last_error()


def test_fused_li_manage_validation():
    from nanovllm_amd import _lib
    from nanovllm_amd._lib import BFLOAT16, INT32

    B = 2

    def descs():
        return [_desc((B, 32, 128), BFLOAT16), _desc((B, 32), BFLOAT16), _desc((8, 128, 1, 128), BFLOAT16),
                _desc((B, 4), INT32), _desc((B,), INT32), _desc((B,), INT32), _desc((B,), INT32),
                _desc((3, 512), INT32), _desc((B, 1, 2048), INT32), _desc((B, 1, 2048), INT32), _desc((B,), INT32)]

    def call(d, ws=0x2000, wsn=1 << 30):
        return _lib.lib.nvdsa_fused_li_manage(*[ctypes.byref(x) for x in d], ws, wsn, None)

    d = descs()
    d[0].shape[1] = 48
    assert call(d) == 1 and "32 or 64" in _lib.last_error()
    d = descs()
    d[7].shape[1] = 500
    assert call(d) == 1 and "state width" in _lib.last_error()
    d = descs()
    d[1].dtype = 3
    assert call(d) == 2 and "dtypes must match" in _lib.last_error()
    d = descs()
    d[8].shape[2] = 1024
    assert call(d) == 1 and "[B, 1, 2048]" in _lib.last_error()
    d = descs()
    assert call(d, ws=0, wsn=0) == 5
    need = _lib.lib.nvdsa_fused_li_manage_workspace_size(B, 512, 32)
    assert need >= B * 512 * 4
    d = descs()
    d[3].shape[1] = 20000
    d[7].shape[1] = 20000 * 128
    assert call(d) == 1 and "16384" in _lib.last_error()


def test_mtp_and_attention_validation():
    from nanovllm_amd import _lib
    from nanovllm_amd._lib import BFLOAT16, INT32

    B = 2
    m = [_desc((4 * B, 32, 128), BFLOAT16), _desc((4 * B, 32), BFLOAT16), _desc((8, 128, 1, 128), BFLOAT16),
         _desc((B, 4), INT32), _desc((B,), INT32), _desc((B,), INT32), _desc((B,), INT32), _desc((3, 512), INT32),
         _desc((4 * B, 1, 2048), INT32), _desc((4 * B, 1, 2048), INT32), _desc((B, 8192), INT32),
         _desc((B, 8192), INT32), _desc((B,), INT32)]
    m[0].shape[0] = 3 * B
    assert _lib.lib.nvdsa_fused_li_manage_mtp(*[ctypes.byref(x) for x in m], 0x2000, 1 << 30, None) == 1
    assert "four packed queries" in _lib.last_error()

    a = [_desc((B, 48, 64), BFLOAT16), _desc((B, 48, 512), BFLOAT16), _desc((B,), INT32), _desc((B,), INT32),
         _desc((B,), INT32), _desc((B, 1, 2048), INT32), _desc((B, 3), INT32), _desc((4, 128, 1, 64), BFLOAT16),
         _desc((4, 128, 1, 512), BFLOAT16)]
    out = _desc((B, 48, 512), BFLOAT16)
    st = _lib.lib.nvdsa_sparse_tail_attention(*[ctypes.byref(x) for x in a], 0.1, ctypes.byref(out), 0x2000,
                                              1 << 30, None)
    assert st == 1 and "power of two" in _lib.last_error()


@pytest.mark.parametrize("mutate,code,msg", [
    (lambda d: setattr(d[0], "ndim", 2), 1, "q_inout rank mismatch."),
    (lambda d: setattr(d[1], "dtype", 1), 2, "cos dtype mismatch."),
    (lambda d: setattr(d[2], "ndim", 3), 1, "sin rank mismatch."),
    (lambda d: setattr(d[2], "contiguous", 0), 3, "sin must be contiguous."),
    (lambda d: [setattr(x, "dtype", 3) for x in d], 2, "float16 or bfloat16"),
    (lambda d: setattr(d[1], "device", 1), 4, "same GPU"),
    (lambda d: d[0].shape.__setitem__(0, 0), 1, "non-empty"),
    (lambda d: d[1].shape.__setitem__(0, 3), 1, "token dimension mismatch"),
    (lambda d: d[0].shape.__setitem__(1, 160), 1, "n_head <= 128"),
    (lambda d: d[0].shape.__setitem__(2, 264), 1, "head_dim <= 256"),
])
def test_query_rope_validation(mutate, code, msg):
    """The reference adapter's checks (dsa_indexer_project_torch_adpt.h:42-90)."""
    from nanovllm_amd import _lib
    from nanovllm_amd._lib import BFLOAT16

    d = [_desc((4, 32, 128), BFLOAT16), _desc((4, 1, 1, 64), BFLOAT16), _desc((4, 1, 1, 64), BFLOAT16)]
    mutate(d)
    assert _lib.lib.nvdsa_dsa_indexer_query_rope_inplace(*[ctypes.byref(x) for x in d], 64, None) == code
    assert msg in _lib.last_error()
    d = [_desc((4, 32, 128), BFLOAT16), _desc((4, 1, 1, 256), BFLOAT16), _desc((4, 1, 1, 256), BFLOAT16)]
    for rope, m in ((48 + 8, "aligned to 16"), (0, "positive"), (144, "no larger than head_dim")):
        assert _lib.lib.nvdsa_dsa_indexer_query_rope_inplace(*[ctypes.byref(x) for x in d], rope, None) == 7
        assert m in _lib.last_error()
    d[1].shape[3] = d[2].shape[3] = 16  # the storage check comes first (adapter order)
    assert _lib.lib.nvdsa_dsa_indexer_query_rope_inplace(*[ctypes.byref(x) for x in d], 64, None) == 1
    assert "storage is smaller" in _lib.last_error()


def test_indexer_project_validation():
    from nanovllm_amd import _lib
    from nanovllm_amd._lib import BFLOAT16, FLOAT32

    T = 3

    def descs():
        return [_desc((T, 6144), BFLOAT16), _desc((T, 2048), BFLOAT16), _desc((T, 1, 1, 64), BFLOAT16),
                _desc((T, 1, 1, 64), BFLOAT16), _desc((4096, 2048), BFLOAT16), _desc((32, 6144), BFLOAT16),
                _desc((T, 32, 128), BFLOAT16), _desc((T, 32), BFLOAT16)]

    def call(d, heads=32, hd=128, rope=64):
        ptrs = [ctypes.byref(x) if x is not None else None for x in d]
        return _lib.lib.nvdsa_dsa_indexer_project_query_only(*ptrs, heads, hd, rope, 1.0, None)

    d = descs()
    d[6].shape[1] = 16
    assert call(d) == 1 and _lib.last_error().endswith("q_index_out shape must be (3, 32, 128), got (3, 16, 128)")
    d = descs()
    d[7].shape[1] = 64
    assert call(d) == 1 and "index_weights_out shape must be (3, 32), got (3, 64)" in _lib.last_error()
    d = descs()
    d[5] = None
    assert call(d) == 7 and "go together" in _lib.last_error()
    d = descs()
    d[1].shape[1] = d[4].shape[1] = 2000
    assert call(d) == 1 and "multiple of 256" in _lib.last_error()
    d = descs()
    d[5].dtype = FLOAT32
    assert call(d) == 2 and "one 16-bit dtype" in _lib.last_error()
    d = descs()
    d[2].shape[3] = d[3].shape[3] = 32
    assert call(d) == 1 and "rope_dim values per token" in _lib.last_error()
    d = descs()
    assert call(d, rope=63) == 7 and "even" in _lib.last_error()
    d = descs()
    d[4].data = 0x1008
    assert call(d) == 3 and "16-byte aligned" in _lib.last_error()


def test_persist_validation():
    from nanovllm_amd import _lib
    from nanovllm_amd._lib import BFLOAT16, FLOAT16, INT32

    def descs():
        return [_desc((8, 128, 512), BFLOAT16), _desc((8, 128, 64), BFLOAT16),
                _desc((16, 128, 1, 512), BFLOAT16, device=-1), _desc((16, 128, 1, 64), BFLOAT16, device=-1),
                _desc((5,), INT32), _desc((5,), INT32)]

    def call(d):
        return _lib.lib.nvdsa_persist_prefill_blocks(*[ctypes.byref(x) for x in d], None)

    d = descs()
    d[0].shape[2] = 256
    assert call(d) == 1 and "CKV caches" in _lib.last_error()
    d = descs()
    d[3].shape[0] = 15
    assert call(d) == 1 and "same number of blocks" in _lib.last_error()
    d = descs()
    d[5].shape[0] = 4
    assert call(d) == 1 and "equal length" in _lib.last_error()
    d = descs()
    d[4].dtype = BFLOAT16
    assert call(d) == 2 and "int32" in _lib.last_error()
    d = descs()
    d[2].dtype = d[3].dtype = FLOAT16
    assert call(d) == 2 and "one 16-bit dtype" in _lib.last_error()
    d = descs()
    d[0].device = -1
    assert call(d) == 4
    d = descs()
    d[1].data = 0x1004
    assert call(d) == 3 and "aligned" in _lib.last_error()


def test_torch_library_schemas_match_reference():
    """Every schema torch registered for nanovllm_dsa hashes to the digest of
    the reference's own string (tests/golden/reference_schemas.json, written
    by tests/golden/make_schema_digests.py from bindings/nanovllm_ops.cpp:645-714),
    and, where the reference checkout is present, equals that string."""
    import hashlib
    import json
    from pathlib import Path

    from nanovllm_amd import ops

    golden = json.loads((Path(__file__).parent / "golden" / "reference_schemas.json").read_text())["sha256"]
    assert set(golden) == set(ops.SCHEMAS)
    registered = {}
    for name in ops.SCHEMAS:
        op = getattr(torch.ops.nanovllm_dsa, name).default
        text = str(op._schema)
        assert text.startswith("nanovllm_dsa::")
        registered[name] = text[len("nanovllm_dsa::"):]
        assert hashlib.sha256(registered[name].encode()).hexdigest() == golden[name], name
    ref = Path("/root/reference")
    if ref.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("make_schema_digests",
                                                      Path(__file__).parent / "golden" / "make_schema_digests.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        theirs = mod.reference_schemas(ref)
        for name, text in registered.items():
            assert theirs[name] == text, name


def test_meta_dispatch_returns_none():
    from nanovllm_amd import dsa_offload_ops as ops

    meta = torch.device("meta")
    bf = torch.bfloat16
    i32 = torch.int32
    out = ops.scatter_copy(torch.empty(2, 16, dtype=i32, device=meta), torch.empty(2, 16, dtype=i32, device=meta),
                           torch.empty(2, dtype=i32, device=meta), torch.empty(2, 2, dtype=i32, device=meta),
                           torch.empty(2, 2, dtype=i32, device=meta), torch.empty(4, 128, 64, dtype=bf, device=meta),
                           torch.empty(4, 128, 512, dtype=bf, device=meta),
                           torch.empty(4, 128, 64, dtype=bf, device=meta),
                           torch.empty(4, 128, 512, dtype=bf, device=meta))
    assert out is None


def test_cpu_tensors_have_no_kernel():
    """No CPU implementation is registered: the oracle is never a fallback."""
    from nanovllm_amd import dsa_offload_ops as ops

    i32 = torch.int32
    with pytest.raises(NotImplementedError):
        ops.scatter_copy(torch.zeros(1, 4, dtype=i32), torch.zeros(1, 4, dtype=i32), torch.zeros(1, dtype=i32),
                         torch.zeros(1, 1, dtype=i32), torch.zeros(1, 1, dtype=i32),
                         torch.zeros(1, 128, 64, dtype=torch.bfloat16), torch.zeros(1, 128, 512, dtype=torch.bfloat16),
                         torch.zeros(1, 128, 64, dtype=torch.bfloat16), torch.zeros(1, 128, 512, dtype=torch.bfloat16))
