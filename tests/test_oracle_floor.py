"""The fp32-order noise floor of the reference semantics, per test configuration.

The reference (engine/model.py:134-242, engine/quantize.py:517-525) fixes every bf16 rounding
point but not the order of the fp32 sums inside a linear, nor the last ulps of the fp32 exp inside
softmax and SiLU. Two valid implementations flip single bf16 roundings, and later bf16 ops spread
the flips, so no implementation can be closer to the oracle than the oracle is to itself under
another valid implementation. These tests measure that distance (max and mean |dlogit|) on
random-KV decode steps and the rows of a batched causal chain, over three summation orders and an
exp2-based softmax / SiLU, and check it against tests/helpers.py's ORDER_FLOOR, from which the GPU
parity bars are built (twice the floor). They also show that the bars are not loose: a misplaced
bf16 rounding point (a plausible kernel mistake) exceeds the all-rows mean bar at one layer.
"""
import os

import pytest
import torch
import torch.nn.functional as F

import oracle.model as om
from flint_amd.synth import CONFIGS, ModelArgs, synth_weights
from tests.helpers import ORDER_FLOOR, agg_bar, log, logit_stats


def _split_rev4(x, w):
    """Reversed 4-way split-K, fp32 partial sums (another valid order)."""
    K = x.shape[-1]
    bs = K // 4
    acc = None
    for b in reversed(range(4)):
        part = x[..., b * bs:(b + 1) * bs].float() @ w[:, b * bs:(b + 1) * bs].float().T
        acc = part if acc is None else acc + part
    return acc.to(x.dtype)


def _chunk32(x, w):
    """fp32 sums of 32-element chunks, then over the chunks (the GEMV kernels' unit of work)."""
    K = x.shape[-1]
    p = (x.float().reshape(*x.shape[:-1], 1, K // 32, 32) * w.float().reshape(w.shape[0], K // 32, 32)).sum(-1)
    return p.sum(-1).to(x.dtype)


# alternative implementations: a linear order alone, or a named oracle implementation (om.IMPLS)
VARIANTS = {"g128": "g128", "rev4": _split_rev4, "chunk32": _chunk32, "exp2": "exp2",
            "g128+exp2": "g128+exp2"}
POSITIONS = {"tiny": (0, 63, 200, 500), "small": (0, 63, 200, 500), "wide": (0, 63, 200, 500),
             "flint-3b-l1": (128, 129, 300, 1000, 2000), "flint-3b": (512, 600, 1024, 8191)}


def _random_kv(a, pos):
    g = torch.Generator().manual_seed(pos + 1)
    k = torch.randn(a.n_layer, a.n_local_heads, pos, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(a.n_layer, a.n_local_heads, pos, 64, generator=g).to(torch.bfloat16)
    return k, v


def _step(o, k, v, pos, variant=None, forward=None):
    """One decode step of token (7 pos + 3) at `pos` over the cache [0, pos) = (k, v), in the
    default implementation or `variant` (a VARIANTS value)."""
    o.setup_caches(pos + 8)
    o.k_cache[:, :, :pos] = k
    o.v_cache[:, :, :pos] = v
    tok = torch.tensor([(7 * pos + 3) % o.args.vocab_size])
    if isinstance(variant, str):
        o.set_order(variant)
    elif variant is not None:
        o.linear = variant
    try:
        lg = (forward or (lambda: o.forward(tok, pos)[0]))()
    finally:
        o.set_order("torch")
    return lg[0].float()


def _chain(o, k, v, pos, m, variant=None):
    """Logits [m, V] of a causal chain of m tokens at pos .. pos+m-1 over the cache [0, pos) =
    (k, v), in one batched forward (the shape of a speculative verify or a prefill chunk)."""
    o.setup_caches(pos + m + 8)
    o.k_cache[:, :, :pos] = k
    o.v_cache[:, :, :pos] = v
    toks = torch.tensor([(7 * (pos + i) + 3) % o.args.vocab_size for i in range(m)])
    if isinstance(variant, str):
        o.set_order(variant)
    elif variant is not None:
        o.linear = variant
    try:
        lg = o.forward(toks, pos)[0]
    finally:
        o.set_order("torch")
    return lg.float()


CHAIN = 24  # rows of the batched chain measured per configuration


def measure_floor(name):
    """Distances between the default implementation and the alternative ones over the rows of
    single decode steps at POSITIONS[name] and of one CHAIN-token batched chain: (largest
    max|dlogit| of a row, largest mean|dlogit| of a row, largest mean|dlogit| over all rows of one
    variant, smallest fraction of a row within 2e-2). A row's mean is heavy-tailed (one flipped
    rounding in the final hidden state moves many logits), the mean over all rows much less so."""
    a = ModelArgs(**CONFIGS[name])
    o = om.OracleModel(a, synth_weights(a, 0))
    worst_max = worst_mean = worst_agg = 0.0
    min_within = 1.0
    rows = {oname: [] for oname in VARIANTS}
    for pos in POSITIONS[name]:
        k, v = _random_kv(a, pos)
        ref = _step(o, k, v, pos)
        for oname, var in VARIANTS.items():
            st = logit_stats(_step(o, k, v, pos, variant=var), ref)
            rows[oname].append(st["mean"])
            log(f"{name} pos={pos} {oname}: max|d|={st['max']:.4f} mean|d|={st['mean']:.3e} "
                f"within 2e-2 {st['within']:.4%}")
            worst_max = max(worst_max, st["max"])
            worst_mean = max(worst_mean, st["mean"])
            min_within = min(min_within, st["within"])
    pos = POSITIONS[name][1]
    k, v = _random_kv(a, pos)
    ref = _chain(o, k, v, pos, CHAIN)
    for oname, var in VARIANTS.items():
        lg = _chain(o, k, v, pos, CHAIN, variant=var)
        for r in range(CHAIN):
            st = logit_stats(lg[r], ref[r])
            rows[oname].append(st["mean"])
            worst_max = max(worst_max, st["max"])
            worst_mean = max(worst_mean, st["mean"])
            min_within = min(min_within, st["within"])
        log(f"{name} chain pos={pos} M={CHAIN} {oname}: row means max {max(rows[oname][-CHAIN:]):.3e} "
            f"avg {sum(rows[oname][-CHAIN:]) / CHAIN:.3e}")
    for oname in VARIANTS:
        worst_agg = max(worst_agg, sum(rows[oname]) / len(rows[oname]))
    return worst_max, worst_mean, worst_agg, min_within


@pytest.mark.parametrize("name", ["tiny", "small", "wide", "flint-3b-l1"])
def test_order_floor(name):
    """Re-measures the recorded floor: no pair of valid implementations differs by more than it."""
    worst_max, worst_mean, worst_agg, min_within = measure_floor(name)
    log(f"{name}: floor max|d| {worst_max:.4f} row mean|d| {worst_mean:.3e} all-rows mean|d| "
        f"{worst_agg:.3e}, within 2e-2 >= {min_within:.4%}")
    fmax, fmean, fagg = ORDER_FLOOR[name]
    assert worst_max <= fmax and worst_mean <= fmean and worst_agg <= fagg
    if name == "flint-3b-l1":
        # one layer of the 3B model: the implementations agree to two bf16 ulps of the top logits
        assert worst_max <= 2.0 ** -4 and min_within >= 0.99


@pytest.mark.slow
def test_order_floor_40_layers():
    """The 40-layer model: the floor grows to about 0.37 (a fifth to a third of the logits within
    2e-2), so the north star's 2e-2 cannot be met even by the reference against itself; the GPU
    bars at 40 layers are twice this. Opt in with FLINT_AMD_SLOW=1 (builds a 6.5 GB oracle)."""
    worst_max, worst_mean, worst_agg, min_within = measure_floor("flint-3b")
    log(f"flint-3b: floor max|d| {worst_max:.4f} row mean|d| {worst_mean:.3e} all-rows mean|d| "
        f"{worst_agg:.3e}, within 2e-2 >= {min_within:.4%}")
    fmax, fmean, fagg = ORDER_FLOOR["flint-3b"]
    assert 0.1 < worst_max <= fmax and worst_mean <= fmean and worst_agg <= fagg
    assert min_within < 0.5


def _slip_forward(o, tok, pos, kind):
    """The oracle forward with ONE planted rounding-point mistake (test-only):
    "act": the SwiGLU product is formed in fp32 and rounded once, instead of
           bf16(bf16(silu(g)) * u) (engine/model.py:227-228);
    "norm": RMSNorm rounds once, bf16(x * rsqrt(..) * w) in fp32, instead of
            bf16(bf16(x * rsqrt(..)) * w) (engine/model.py:237-242)."""
    a = o.args
    lin = o.linear
    x = o.embed[tok.long()] * a.embedding_multiplier
    for l in range(o.L):
        w = o.w[l]
        h1 = x + o.layer_attention(l, x, pos) * a.residual_multiplier
        if kind == "norm":
            hf = h1.float()
            hn = (hf * torch.rsqrt((hf * hf).mean(-1, keepdim=True) + a.norm_eps) *
                  w["ffn_norm"].float()).to(torch.bfloat16)
        else:
            hn = om.rms_norm(h1, w["ffn_norm"], a.norm_eps)
        if kind == "act":
            act = (F.silu(lin(hn, w["w1"]).float()) * lin(hn, w["w3"]).float()).to(torch.bfloat16)
        else:
            act = F.silu(lin(hn, w["w1"])) * lin(hn, w["w3"])
        x = h1 + lin(act, w["w2"]) * a.residual_multiplier
    return lin(om.rms_norm(x, o.norm, a.norm_eps), o.embed) / a.logits_scaling


@pytest.mark.parametrize("kind", ["act", "norm"])
def test_bars_catch_a_misplaced_rounding(kind):
    """At one layer of the 3B model the parity bars reject a single misplaced bf16 rounding: over
    the steps of a check it raises mean|dlogit| above agg_bar (the bar on the mean over all rows),
    while every valid implementation stays inside."""
    name = "flint-3b-l1"
    a = ModelArgs(**CONFIGS[name])
    o = om.OracleModel(a, synth_weights(a, 0))
    means = []
    for pos in (128, 300, 1000):
        k, v = _random_kv(a, pos)
        tok = torch.tensor([(7 * pos + 3) % a.vocab_size])
        ref = _step(o, k, v, pos)
        st = logit_stats(_step(o, k, v, pos, forward=lambda: _slip_forward(o, tok, pos, kind)), ref)
        log(f"planted {kind} pos={pos}: max|d|={st['max']:.4f} mean|d|={st['mean']:.3e} "
            f"within 2e-2 {st['within']:.4%}")
        means.append(st["mean"])
    agg = sum(means) / len(means)
    log(f"planted {kind}: mean over the steps {agg:.3e} (bar {agg_bar(name):.2e})")
    assert agg > agg_bar(name)


@pytest.mark.slow
def test_flip_counts_at_40_layers():
    """Greedy argmax flips over 64 steps at 40 layers, on the oracle alone: its own greedy tokens
    after its own 511-token prefill (seeded uniform prompt), each step also run in the three other
    valid implementations and with each planted rounding slip of _slip_forward, flips counted
    against the default implementation. At this depth the slips flip no more often than the valid
    implementations do (a flip count cannot tell a misplaced rounding point from order noise),
    which is why the GPU tests also check every layer on its own. Opt in with FLINT_AMD_SLOW=1."""
    a = ModelArgs(**CONFIGS["flint-3b"])
    o = om.OracleModel(a, synth_weights(a, 0))
    o.setup_caches(1024)
    g = torch.Generator().manual_seed(512)
    prompt = torch.randint(0, a.vocab_size, (512,), generator=g, dtype=torch.int32)
    for b in range(0, 511, 64):
        o.forward(prompt[b:min(511, b + 64)], b)

    def run(tok, pos, impl=None, slip=None):
        if slip:
            return _slip_forward(o, tok, pos, slip)[0].float()
        o.set_order(impl or "torch")
        try:
            return o.forward(tok, pos)[0][0].float()
        finally:
            o.set_order("torch")
    names = [("g128", "g128", None), ("exp2", "exp2", None), ("g128+exp2", "g128+exp2", None),
             ("slip act", None, "act"), ("slip norm", None, "norm")]
    flips = {n: 0 for n, _, _ in names}
    cur = int(prompt[511])
    for i in range(64):
        tok, pos = torch.tensor([cur]), 511 + i
        others = {n: run(tok, pos, impl, slip) for n, impl, slip in names}  # before the default: it
        ref = run(tok, pos)                                                 # writes the cache last
        am = int(torch.argmax(ref))
        for n, lg in others.items():
            flips[n] += int(torch.argmax(lg)) != am
        cur = am
    log(f"40-layer argmax flips over 64 steps against the default implementation: {flips}")
    valid = max(flips[n] for n in ("g128", "exp2", "g128+exp2"))
    assert max(flips["slip act"], flips["slip norm"]) <= valid + 4
