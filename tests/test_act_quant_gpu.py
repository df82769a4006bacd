"""GPU parity of the per-row quantiser (int8 and fp8 e4m3fn) against the oracle, and of
the fp8 indexer fed by it.

Bit-exact: int8 codes, fp8 codes and scales equal the oracle's restatement of
act_quant_torch (examples/deepseek_v4/act_quant.py:118-142) for bf16 / fp16 /
fp32 inputs, with and without round_scale, aligned and ragged rows.  The fp8
indexer on quantised q / k (key scale as key_scale, query scale folded into the
head weights) matches the oracle's logits of the dequantised inputs within the
indexer tolerance (1e-2 relative).
"""
import pytest
import torch

from oracle import dsa_oracle as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.int8, torch.float8_e4m3fn])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("round_scale", [False, True])
def test_codes_and_scales_bit_exact(dsa, dev, dtype, xdtype, round_scale):
    g = torch.Generator().manual_seed(3)
    for shape in ((37, 7168), (5, 128), (3, 4, 96), (9, 13), (2, 1)):
        x = (torch.randn(shape, generator=g) * 3).to(xdtype)
        x.view(-1, shape[-1])[0].zero_()                     # an all-zero row: the 1e-4 floor
        y, s = dsa.act_quant(x.to(dev), round_scale=round_scale, dtype=dtype)
        wy, ws = ref.act_quant(x, round_scale=round_scale, dtype=dtype)
        assert y.shape == x.shape and s.shape == x.shape[:-1] + (1,)
        assert torch.equal(s.cpu(), ws), shape
        assert torch.equal(y.cpu().view(torch.uint8), wy.view(torch.uint8)), shape


def test_fp8_indexer_from_quantised_inputs(dsa, dev):
    g = torch.Generator().manual_seed(4)
    B, S1, S2, H, D = 1, 64, 1500, 64, 128
    qf = torch.randn(B, S1, H, D, generator=g).to(torch.bfloat16)
    kf = torch.randn(B, S2, D, generator=g).to(torch.bfloat16)
    w = torch.randn(B, S1, H, generator=g) / 8
    q8, qs = dsa.act_quant(qf.view(B * S1 * H, D).to(dev), dtype=torch.float8_e4m3fn)
    k8, ks = dsa.act_quant(kf.view(B * S2, D).to(dev), dtype=torch.float8_e4m3fn)
    got = dsa.indexer_logits(q8.view(B, S1, H, D), k8.view(B, S2, 1, D), w.to(dev), ks.view(B, S2),
                             query_scale=qs.view(B, S1, H), sparse_mode=3).cpu()
    # The oracle on the dequantised values: q8 * qs and k8 * ks.
    qd = (q8.float() * qs).cpu().view(B, S1, H, D)
    kd = k8.float().cpu().view(B, S2, D)
    want = ref.indexer_logits(qd, kd, w, ks.cpu().view(B, S2), sparse_mode=3)
    fin = torch.isfinite(want)
    assert torch.equal(fin, torch.isfinite(got))
    rms = want[fin].double().pow(2).mean().sqrt().item()
    assert torch.all((got[fin] - want[fin]).abs() <= 1e-2 * (want[fin].abs() + rms))
    # Against the unquantised bf16 inputs the fp8 rounding stays small.
    full = ref.indexer_logits(qf, kf, w, None, sparse_mode=3)
    assert ((got[fin] - full[fin]).abs().mean() / full[fin].abs().mean()).item() < 0.1
