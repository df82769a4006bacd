"""CPU checks of the torch.ops.dsa registrations: schemas and Meta (shape-only)
implementations, the pattern of examples/torch_tl_ascend/src/_inner.cpp:58-68."""
import torch


def test_schemas_registered(dsa):
    ops = dsa.load_torch_ops()
    for name in ("topk_select", "lightning_indexer", "sparse_mla_fwd", "sparse_flash_mla", "act_quant",
                 "sparse_attn"):
        assert getattr(ops, name).default._schema.name == f"dsa::{name}"


def test_meta_shapes(dsa):
    ops = dsa.load_torch_ops()
    m = dict(device="meta")
    i, v = ops.topk_select(torch.empty(6, 1000, **m), 64)
    assert i.shape == (6, 64) and i.dtype == torch.int32 and v.shape == (6, 64)
    i, v = ops.lightning_indexer(torch.empty(2, 5, 64, 128, dtype=torch.float8_e4m3fn, **m),
                                 torch.empty(2, 300, 1, 128, dtype=torch.float8_e4m3fn, **m),
                                 torch.empty(2, 5, 64, **m), sparse_count=128, return_value=True)
    assert i.shape == (2, 5, 1, 128) and v.shape == (2, 5, 1, 128)
    o, l = ops.sparse_mla_fwd(torch.empty(1, 4, 16, 576, dtype=torch.bfloat16, **m),
                              torch.empty(1, 64, 1, 576, dtype=torch.bfloat16, **m),
                              torch.empty(1, 4, 1, 32, dtype=torch.int32, **m), 0.05)
    assert o.shape == (1, 4, 16, 512) and o.dtype == torch.bfloat16 and l.shape == (1, 4, 16)
    o, l = ops.sparse_flash_mla(torch.empty(7, 64, 512, dtype=torch.bfloat16, **m),
                                torch.empty(4, 128, 1, 512, dtype=torch.bfloat16, **m),
                                torch.empty(1, 4, dtype=torch.int32, **m), torch.empty(1, dtype=torch.int32, **m),
                                torch.empty(1, dtype=torch.int32, **m), torch.empty(1, dtype=torch.int32, **m),
                                torch.empty(64, **m), 0.04)
    assert o.shape == (7, 64, 512) and l.shape == (7, 64)
    y, s = ops.act_quant(torch.empty(3, 5, 128, dtype=torch.bfloat16, **m), False, torch.float8_e4m3fn)
    assert y.shape == (3, 5, 128) and y.dtype == torch.float8_e4m3fn and s.shape == (3, 5, 1)
    y, s = ops.act_quant(torch.empty(4, 64, **m))
    assert y.dtype == torch.int8 and s.shape == (4, 1)
    o, l = ops.sparse_attn(torch.empty(1, 6, 16, 512, dtype=torch.bfloat16, **m),
                           torch.empty(1, 9, 512, dtype=torch.bfloat16, **m), torch.empty(16, **m),
                           torch.empty(1, 6, 4, dtype=torch.int32, **m), 0.04)
    assert o.shape == (1, 6, 16, 512) and o.dtype == torch.float32 and l.shape == (1, 6, 16)
