"""MI355X (gfx950) implementation of the DSA stable-decode offload chain.

``import nanovllm_amd.ops`` registers ``torch.ops.nanovllm_dsa.*`` (the
reference's operator namespace) backed by the HIP library ``libnvdsa.so``;
``nanovllm_amd.dsa_offload_ops`` holds the caller-side wrappers with the
reference's signatures.
"""

LIDU_TOPK = 2048
LIDU_MTP_QUERY_COUNT = 4
LIDU_MTP_UNION_CAPACITY = LIDU_TOPK * LIDU_MTP_QUERY_COUNT
BLOCK_SIZE = 128
CKV_DIM = 512
KPE_DIM = 64
INDEX_DIM = 128

__all__ = [
    "LIDU_TOPK",
    "LIDU_MTP_QUERY_COUNT",
    "LIDU_MTP_UNION_CAPACITY",
    "BLOCK_SIZE",
    "CKV_DIM",
    "KPE_DIM",
    "INDEX_DIM",
]
