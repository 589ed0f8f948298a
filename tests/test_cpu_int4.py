"""Pins the timed CPU baseline (oracle/cpu_int4.py: the reference int4 decode path with torch's
CPU int4 kernel) against the oracle.

torch's aten::_weight_int4pack_mm_for_cpu takes the same int4 values and [K/128, N, 2] scales and
zeros as gpt-fast's linear (engine/quantize.py:359-373, 517-525) but does not round the
dequantised weight twice as gpt-fast's Python definition does (quantize.py:152-154). So:
  * per linear, a closed-form bound: each weight may differ by one bf16 ulp of the larger of
    bf16((q - 8) * s) and the dequantised value, so |y - y_oracle| <= sum_k |x_k| * that ulp +
    one output ulp on each side; a packing mistake (scales and zeros swapped) breaks it;
  * per decode step (and the prefill's next token), the logits stay within a bar twice the
    largest distance measured at up to four layers (max 0.094, mean 0.0196) and the greedy token
    equals the oracle's except where the oracle's top-2 margin is within that bar.
"""
import pytest
import torch

from flint_amd.synth import CONFIGS, ModelArgs, synth_weights
from oracle import quant
from oracle.cpu_int4 import CpuInt4Decoder, CpuInt4Linear
from oracle.model import OracleModel
from tests.helpers import log, logit_stats, near_tie, top2_margin

CPU_BAR_MAX = 0.1875
CPU_BAR_MEAN = 0.04


def _ulp(t):
    m = t.float().abs().clamp(min=2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(m)) - 7)


def _bound(x, w, y, yr):
    q, s, z = quant.group_quantize(w)
    dq = quant.group_dequantize(q, s, z)
    p = (q.reshape(-1, quant.GROUP) - 8).mul(s.reshape(-1, 1)).reshape(q.shape)  # bf16((q-8)*s)
    dw = torch.maximum(_ulp(p), _ulp(dq))
    return x.float().abs() @ dw.T + _ulp(y) + _ulp(yr)


@pytest.mark.parametrize("n,k", [(512, 512), (3584, 2560), (2560, 8192)])
def test_cpu_int4_linear_within_dequant_bound(n, k):
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(4, k, generator=g).to(torch.bfloat16)
    lin = CpuInt4Linear(w)
    y = lin(x).float()
    yr = torch.nn.functional.linear(x, quant.dq_linear_weight(w)).float()
    B = _bound(x, w, y, yr)
    r = float(((y - yr).abs() / B).max())
    log(f"int4 CPU linear {n}x{k}: max |y - y_oracle| / bound = {r:.3f}")
    assert r <= 1.0
    # planted packing mistake: scales and zeros swapped in the [K/128, N, 2] tensor
    lin.sz = lin.sz.flip(-1).contiguous()
    assert float(((lin(x).float() - yr).abs() / B).max()) > 1.0


@pytest.mark.parametrize("name", ["tiny", "small", "flint-3b-l1"])
def test_cpu_int4_decoder_matches_oracle(name):
    a = ModelArgs(**CONFIGS[name])
    sd = synth_weights(a, 0)
    dec, orc = CpuInt4Decoder(a, sd), OracleModel(a, sd)
    P = 40
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, a.vocab_size, (P + 8,), generator=g)
    dec.setup_caches(P + 16)
    orc.setup_caches(P + 16)
    nt = dec.prefill(prompt[:P], chunk=16)
    lo, _ = orc.forward(prompt[:P], 0)
    assert nt == int(torch.argmax(lo[-1])) or near_tie(lo[-1], CPU_BAR_MAX)
    for i in range(8):
        ld = dec.step_logits(int(prompt[P + i]), P + i).float()
        lr = orc.forward(prompt[P + i:P + i + 1], P + i)[0][0].float()
        st = logit_stats(ld, lr)
        log(f"{name} step {i}: max|d|={st['max']:.4f} mean|d|={st['mean']:.2e} within 2e-2 {st['within']:.2%} "
            f"argmax {int(ld.argmax())}/{int(lr.argmax())} margin {top2_margin(lr):.4f}")
        assert st["max"] <= CPU_BAR_MAX and st["mean"] <= CPU_BAR_MEAN
        assert int(ld.argmax()) == int(lr.argmax()) or near_tie(lr, CPU_BAR_MAX)
