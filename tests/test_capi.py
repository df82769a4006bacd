"""CPU checks of the boundary: the library loads, exports every symbol declared
in include/*.h, and rejects bad arguments (no kernel is launched)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(dsa_[A-Za-z0-9_]+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert {"dsa_topk_select", "dsa_topk_select_ws", "dsa_topk_select_workspace_size", "dsa_indexer_logits",
            "dsa_lightning_indexer", "dsa_sparse_mla_fwd", "dsa_sparse_mla_workspace_size",
            "dsa_lightning_indexer_workspace_size"} <= names


def test_library_exports_every_declared_symbol(dsa):
    lib = ctypes.CDLL(str(dsa.library_path()))
    missing = [n for n in sorted(_declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_signatures_cover_the_header(dsa):
    from importlib import import_module
    lib_mod = import_module("tilelang_ascend_amd._lib")
    assert set(lib_mod.SIGNATURES) == _declared_functions()


def test_abi_rejects_bad_arguments_without_launching(dsa):
    lib = dsa.load_library()
    assert lib.dsa_abi_version() == 106
    # k out of range
    assert lib.dsa_topk_select(None, 8, 1, 8, 0, None, 1, None, None, None) == 1
    assert b"k must be" in lib.dsa_last_error_message()
    # indexer: bad head dim
    assert lib.dsa_indexer_logits(0, None, None, None, None, 1, 1, 1, 16, 96, None, None, None, 0, 0, 3, None, 1,
                                  None) == 1
    assert b"head dim" in lib.dsa_last_error_message()
    # sparse MLA: wrong dims
    assert lib.dsa_sparse_mla_fwd(1, None, None, None, None, None, None, 1, 1, 16, 512, 512, 16, 0, 0, 16, 1.0, 1,
                                  None, None, None, 0, None) == 1
    assert b"d_qk" in lib.dsa_last_error_message()
    # sparse MLA: workspace too small when the index list is split
    need = lib.dsa_sparse_mla_workspace_size(1, 1, 128, 2048)
    assert need > 0
    assert lib.dsa_sparse_mla_fwd(1, 8, 8, 8, None, None, None, 1, 1, 128, 576, 512, 4096, 0, 0, 2048, 1.0, 1,
                                  8, 8, None, need - 1, None) == 1
    assert b"workspace" in lib.dsa_last_error_message()


def test_python_layer_refuses_cpu_tensors(dsa):
    x = torch.randn(4, 64)
    with pytest.raises(ValueError, match="HIP"):
        dsa.topk_selector(x, 8)
    q = torch.zeros(1, 2, 16, 576, dtype=torch.bfloat16)
    kv = torch.zeros(1, 8, 1, 576, dtype=torch.bfloat16)
    idx = torch.zeros(1, 2, 1, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="HIP"):
        dsa.sparse_mla_fwd(q, kv, idx)


def test_grouped_sparse_attention_host_logic(dsa):
    """dsa_sparse_attention_fwd: workspace sizes and argument checks (host only)."""
    lib = dsa.load_library()
    # kv_group 1 asks for what dsa_sparse_mla_fwd asks for; G groups of H / G heads for the
    # split partials of B * S * G rows; the 128-wide kernel needs none.
    for B, S, H, k in ((1, 1, 128, 2048), (2, 64, 128, 2048), (1, 4, 16, 512)):
        assert (lib.dsa_sparse_attention_workspace_size(B, S, H, 1, 576, k)
                == lib.dsa_sparse_mla_workspace_size(B, S, H, k))
    assert (lib.dsa_sparse_attention_workspace_size(1, 1, 128, 2, 576, 2048)
            == lib.dsa_sparse_mla_workspace_size(1, 2, 64, 2048))
    assert lib.dsa_sparse_attention_workspace_size(2, 273, 64, 4, 128, 2048) == 0
    assert lib.dsa_sparse_attention_workspace_size(1, 1, 100, 3, 576, 2048) == 0  # H % G != 0

    def call(H, G, d_qk, d_v, topk=2048, bt=None, Skv=4096, kind=1):
        return lib.dsa_sparse_attention_fwd(kind, 8, 8, 8, bt, None, None, 1, 1, H, G, d_qk, d_v, Skv, 64, 4, topk,
                                            1.0, 1, 8, 8, None, 0, None)

    assert call(64, 3, 128, 128) == 1 and b"multiple of kv_group" in lib.dsa_last_error_message()
    assert call(96, 4, 576, 512) == 1 and b"multiple of 16" in lib.dsa_last_error_message()
    assert call(64, 4, 128, 128, topk=8193) == 1 and b"8192" in lib.dsa_last_error_message()
    assert call(64, 4, 128, 128, bt=8) == 1 and b"block table" in lib.dsa_last_error_message()
    assert call(64, 4, 256, 256) == 1 and b"(576, 512) or (128, 128)" in lib.dsa_last_error_message()
    assert call(64, 4, 128, 128, Skv=1 << 29) == 1 and b"2^31" in lib.dsa_last_error_message()
    assert call(64, 4, 128, 128, kind=3) == 1 and b"kind" in lib.dsa_last_error_message()


def test_python_layer_validation_messages(dsa):
    q = torch.zeros(1, 2, 16, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="sparse_count"):
        dsa.lightning_indexer(q, q, torch.zeros(1, 2, 16), sparse_count=3000)
    with pytest.raises(ValueError, match="sparse_mode"):
        dsa.lightning_indexer(q, q, torch.zeros(1, 2, 16), sparse_mode=1)
    with pytest.raises(ValueError, match="dtype"):
        dsa.lightning_indexer(q, q.to(torch.bfloat16), torch.zeros(1, 2, 16))
    with pytest.raises(ValueError, match="non-casual|non-causal"):
        dsa.sparse_attention_fwd(128, 512, 64, 2048, is_causal=False)


def test_fused_indexer_host_logic(dsa):
    """When the fused indexer applies, its workspace, and its argument checks (host only)."""
    lib = dsa.load_library()
    # C2 and C5 rows apply, up to the reference's largest sparse_count (8192, a multiple of
    # 1024: lightning_indexer.py:1238-1239); short rows and S2 < 8k do not.
    assert lib.dsa_lightning_indexer_fused_applies(1, 4096, 32768, 2048) == 1
    assert lib.dsa_lightning_indexer_fused_applies(1, 4096, 131072, 2048) == 1
    assert lib.dsa_lightning_indexer_fused_applies(32, 1, 131072, 2048) == 1
    for k in (6144, 8192):
        assert lib.dsa_lightning_indexer_fused_applies(1, 4096, 131072, k) == 1
    assert lib.dsa_lightning_indexer_fused_applies(1, 4096, 32768, 8192) == 0
    assert lib.dsa_lightning_indexer_fused_applies(1, 4096, 8192, 2048) == 0
    assert lib.dsa_lightning_indexer_fused_applies(1, 64, 20000, 4096) == 0
    # The fused workspace holds no dense logits: flagged rows are recomputed in rounds in a
    # bounded buffer.  At C5 (4096 x 131072, k = 2048) it is well under half the dense path's,
    # whose logits alone take 2 GiB; at k = 8192 it stays under the dense path's too.
    dense = lib.dsa_lightning_indexer_workspace_size(1, 4096, 131072, 2048)
    fused = lib.dsa_lightning_indexer_fused_workspace_size(1, 4096, 131072, 2048)
    assert dense >= 4096 * 131072 * 4 and 0 < fused < dense // 2
    assert (lib.dsa_lightning_indexer_fused_workspace_size(1, 4096, 131072, 8192)
            < lib.dsa_lightning_indexer_workspace_size(1, 4096, 131072, 8192))
    # Where the fused path does not apply the entry runs the dense path and asks for exactly
    # its workspace.
    assert (lib.dsa_lightning_indexer_fused_workspace_size(1, 16, 4096, 2048)
            == lib.dsa_lightning_indexer_workspace_size(1, 16, 4096, 2048))
    assert lib.dsa_lightning_indexer_tnd_fused_workspace_size(2, 100, 80, 40000, 2048) > 0
    # Argument checks, before any launch.
    assert lib.dsa_lightning_indexer_fused(0, 8, 8, None, 8, 1, 16, 32768, 64, 128, None, None, None, 0, 0, 3,
                                           0, 8, None, 8, 1 << 40, None) == 1
    assert b"sparse_count" in lib.dsa_last_error_message()
    assert lib.dsa_lightning_indexer_fused(0, 8, 8, None, 8, 1, 16, 32768, 64, 128, None, None, None, 0, 0, 3,
                                           2048, 8, None, 8, 16, None) == 1
    assert b"workspace" in lib.dsa_last_error_message()
    assert lib.dsa_lightning_indexer_tnd_fused(0, 8, 8, None, 8, 1, 16, 16, 32768, 64, 128, None, 8, None, None,
                                               0, 0, 3, 2048, 8, None, 8, 1 << 40, None) == 1
    assert b"cu_q" in lib.dsa_last_error_message()
    assert lib.dsa_lightning_indexer_fused_fallback_rows(8, 1, 16, 4096, 2048, 8, None) == 1
    assert b"does not apply" in lib.dsa_last_error_message()


def test_sparse_attn_sink_host_checks(dsa):
    lib = dsa.load_library()
    args = lambda kind, H, D: (kind, 8, 8, 8, 1, 4, H, 16, D, 8, None, 0.1, 8, 8, 8, 1 << 30, None)
    assert lib.dsa_sparse_attn_sink(*args(0, 64, 512)) == 1
    assert b"kind" in lib.dsa_last_error_message()
    assert lib.dsa_sparse_attn_sink(*args(1, 64, 576)) == 1
    assert b"D must be 512" in lib.dsa_last_error_message()
    assert lib.dsa_sparse_attn_sink(*args(1, 40, 512)) == 1
    assert b"multiple of 16" in lib.dsa_last_error_message()
    assert lib.dsa_sparse_attn_sink_workspace_size(1, 4, 64, 8) > 0
