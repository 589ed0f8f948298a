"""The CPU oracle against golden vectors of the reference forward itself.

tests/golden/tiny_forward.pt was written by tests/golden/make_golden.py, which ran the
reference's engine/model.py Transformer (a 5-token prefill, then 3 decode steps) on a tiny
configuration with non-default Granite multipliers. The oracle (which the GPU kernels are
tested against) must reproduce it: the same bf16 rounding points in the same order, so logits
equal up to fp32 summation order inside attention (the reference calls SDPA, whose CPU kernel
blocks the key loop; the oracle runs an explicit fp32 softmax, the math-path semantics): at
these sizes that is below 1e-3 on logits of magnitude 0.7. A plausible restatement mistake (a
dropped multiplier, a rounding point moved, the RoPE pair convention or the GQA head map wrong)
changes logits by far more than that.
"""
import os

import torch

from flint_amd.synth import ModelArgs, synth_weights
from oracle.model import OracleModel

HERE = os.path.dirname(os.path.abspath(__file__))


def _load():
    fx = torch.load(os.path.join(HERE, "golden", "tiny_forward.pt"), weights_only=True)
    args = ModelArgs(**fx["config"])
    sd = synth_weights(args, seed=fx["seed"])
    import importlib.util
    spec = importlib.util.spec_from_file_location("mk", os.path.join(HERE, "golden", "make_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    assert mk.weights_digest(sd) == fx["weights_sha256"], "synthetic weights drifted from the fixture"
    return fx, args, sd


def test_oracle_matches_reference_forward():
    fx, args, sd = _load()
    orc = OracleModel(args, sd)
    orc.setup_caches(args.block_size)
    worst = 0.0
    for st in fx["steps"]:
        lo, ho = orc.forward(st["tokens"], st["pos"])
        d = (lo.float() - st["logits"].float()).abs()
        worst = max(worst, float(d.max()))
        assert torch.equal(torch.argmax(lo, dim=-1), torch.argmax(st["logits"], dim=-1))
        # post-norm feature: within one bf16 ulp of its largest element
        dh = float((ho.float() - st["hidden"].float()).abs().max())
        assert dh <= float(st["hidden"].float().abs().max()) * 2.0 ** -7, dh
    print(f"golden: worst |dlogit| {worst:.3e}")
    # measured 9.8e-4 (|logits| <= 0.71): fp32 order inside the softmax only; the single-token
    # step is bit-equal when the oracle calls SDPA itself
    assert worst <= 4e-3


def test_golden_detects_a_planted_mistake():
    """The fixture pins the multipliers: the oracle with the residual multiplier dropped fails."""
    fx, args, sd = _load()
    bad = ModelArgs(**{**fx["config"], "residual_multiplier": 1.0})
    orc = OracleModel(bad, sd)
    orc.setup_caches(args.block_size)
    st = fx["steps"][0]
    lo, _ = orc.forward(st["tokens"], st["pos"])
    assert float((lo.float() - st["logits"].float()).abs().max()) > 2e-2
