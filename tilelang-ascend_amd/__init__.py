"""MI355X (gfx950) DeepSeek Sparse Attention path: lightning indexer -> top-k -> sparse MLA.

Hand-written HIP kernels behind the C ABI of ``include/dsa_mi355x.h``; this
package is the host-side mirror of the reference's Python operator interface
(examples/lightning_indexer, examples/topk_selector,
examples/sparse_flash_attention and examples/deepseek_v4 of tilelang-ascend,
including the V4 ``sparse_flash_mla`` operator).
"""
from ._lib import DSAError, library_path, load_library, load_torch_ops
from .act_quant import act_quant
from .lightning_indexer import indexer, indexer_logits, lightning_indexer
from .sparse_flash_mla import sparse_attn, sparse_attn_kernel, sparse_flash_mla
from .sparse_mla import sparse_attention_fwd, sparse_attn_tilelang, sparse_gqa_fwd, sparse_mla_fwd
from .topk_selector import simple_topk_selector, topk_selector

__all__ = [
    "DSAError",
    "act_quant",
    "indexer",
    "indexer_logits",
    "library_path",
    "lightning_indexer",
    "load_library",
    "load_torch_ops",
    "simple_topk_selector",
    "sparse_attention_fwd",
    "sparse_attn",
    "sparse_attn_kernel",
    "sparse_attn_tilelang",
    "sparse_flash_mla",
    "sparse_gqa_fwd",
    "sparse_mla_fwd",
    "topk_selector",
]
