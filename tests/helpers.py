"""Shared helpers of the parity tests: build engine + oracle from the same seeded weights."""
import sys

import torch

from flint_amd.synth import ModelArgs, synth_weights


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_pair(name, seed=0, n_layer=None, device="cuda", weight_device="cpu", **over):
    """(args, sd, engine, oracle) for config `name` with identical bf16 master weights."""
    from flint_amd.model import Transformer
    from oracle.model import OracleModel
    cfg = dict(**__import__("flint_amd.synth", fromlist=["CONFIGS"]).CONFIGS[name])
    if n_layer is not None:
        cfg["n_layer"] = n_layer
    cfg.update(over)
    args = ModelArgs(**cfg)
    sd = synth_weights(args, seed, device=weight_device)
    eng = Transformer.from_weights(args, sd, device)
    orc = OracleModel(args, {k: v.cpu() for k, v in sd.items()})
    return args, sd, eng, orc


def fill_kv_random(eng, orc, npos, seed=1):
    """Fill cache slots [0, npos) of both engine and oracle with the same bf16 N(0,1) values."""
    g = torch.Generator().manual_seed(seed)
    shape = eng.k_cache.shape
    k = torch.randn(shape[0], shape[1], npos, shape[3], generator=g).to(torch.bfloat16)
    v = torch.randn(shape[0], shape[1], npos, shape[3], generator=g).to(torch.bfloat16)
    eng.k_cache[:, :, :npos] = k.to(eng.k_cache.device)
    eng.v_cache[:, :, :npos] = v.to(eng.v_cache.device)
    orc.k_cache[:, :, :npos] = k
    orc.v_cache[:, :, :npos] = v


def top2_margin(logits):
    v = torch.topk(logits.float(), 2).values
    return float(v[0] - v[1])


def bf16_ulp(v):
    """ulp of a bf16 value of magnitude |v| (elementwise, v fp32 tensor)."""
    a = v.abs().clamp(min=2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - 7)


# fp32 summation-order noise floor of the reference semantics: two valid fp32 orders of the
# CPU oracle itself differ by up to 0.03-0.06 in logits at the 3B model's dimensions (measured,
# tests/test_oracle.py::test_fp32_order_noise_floor); the bar is twice the largest measured.
NOISE_FLOOR = 0.125
NORTH_STAR_TOL = 2e-2


def near_tie(ref_logits, margin=NOISE_FLOOR):
    """True when the reference's top-2 logits are closer than the fp32-order noise floor, so the
    argmax is not determined by the reference semantics themselves."""
    v = torch.topk(ref_logits.float(), 2).values
    return float(v[0] - v[1]) <= margin


def compare_logits(eng, ref):
    """(ok, max|d|, fraction of logits within 2e-2, fraction bit-identical)."""
    e, r = eng.float(), ref.float()
    d = (e - r).abs()
    return (bool((d <= NOISE_FLOOR).all()), float(d.max()),
            float((d <= NORTH_STAR_TOL).float().mean()), float((d == 0).float().mean()))
