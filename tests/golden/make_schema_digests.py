"""Write tests/golden/reference_schemas.json: the SHA-256 of each operator
schema string the reference registers (bindings/nanovllm_ops.cpp:645-714,
``TORCH_LIBRARY(nanovllm_dsa, ops)``), for the operators this build
registers.  Run in a container where the reference checkout is present:

    python tests/golden/make_schema_digests.py [/root/reference]

Only digests are written (no source text): the CPU test hashes the schema
strings torch registered for ``nanovllm_amd`` and compares."""

from __future__ import annotations

import hashlib
import json
import re
import sys
from pathlib import Path

OPS = ("fused_li_manage", "fused_li_manage_mtp", "scatter_copy", "sparse_tail_attention",
       "sparse_tail_attention_mtp", "fused_copy_sfa", "fused_copy_sfa_mtp", "dsa_indexer_query_rope_inplace")
BINDINGS = "csrc/nanovllm_ascend_ops/bindings/nanovllm_ops.cpp"


def reference_schemas(root: Path) -> dict:
    """{op name: schema string} of every ``ops.def("...")`` in the bindings,
    the adjacent C++ string literals joined."""
    text = (root / BINDINGS).read_text()
    out = {}
    for m in re.finditer(r"ops\.def\(\s*((?:\"(?:[^\"\\]|\\.)*\"\s*)+)\)", text):
        schema = "".join(re.findall(r"\"((?:[^\"\\]|\\.)*)\"", m.group(1)))
        out[schema.split("(", 1)[0]] = schema
    return out


def main() -> int:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    schemas = reference_schemas(root)
    digests = {op: hashlib.sha256(schemas[op].encode()).hexdigest() for op in OPS}
    out = Path(__file__).with_name("reference_schemas.json")
    out.write_text(json.dumps({"source": BINDINGS, "sha256": digests}, indent=1) + "\n")
    print(f"wrote {out} ({len(digests)} schemas)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
