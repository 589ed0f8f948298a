"""Parity at the benchmark's own sizes: the 3B-class model's layer shape (config 0), the full
40-layer model in greedy decode at context 512 (config 2) and 8192 (config 3), and speculative
verify at context 1024 (config 4), each against the CPU oracle on the same weights and cache.

Bars (tests/helpers.py row_bars): each step's max and mean |dlogit| within twice the oracle's own
floor, the larger of the model's recorded floor (one layer: 0.047 / 5.6e-3; 40 layers: 0.37 /
6.3e-2, where the oracle agrees with itself on only a quarter to a third of the logits within 2e-2)
and the distance of the oracle's second implementation (per-group summation order, exp2-based
softmax / SiLU) on the same step, which is logged beside every kernel figure. Greedy argmax must
equal the oracle's except where the oracle's top-2 margin is within the max bar.

The 40-layer oracle cannot prefill hundreds of tokens on the CPU in a test's time, so the prompt is
prefilled by the engine (the verify kernel, 32 tokens per launch; its own parity is tested in
test_gpu_verify.py and below) and the resulting K/V rows are copied into the oracle's cache: every
compared step then starts from the same cache on both sides, and from there each side writes its
own rows (teacher forcing on the engine's tokens).
"""
import math
import time

import pytest
import torch

from flint_amd.synth import ModelArgs, synth_weights
from tests.helpers import (bf16_ulp, log, logit_bar, logit_stats, near_tie, oracle_pair, record, say,
                           row_bars, top2_margin, ulp_stats)

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

FULL = "flint-3b"
L1 = "flint-3b-l1"


def _build(name, seed, max_seq):
    from flint_amd.model import Transformer
    from oracle.model import OracleModel
    args = ModelArgs.from_name(name)
    t0 = time.time()
    sd = synth_weights(args, seed, device="cuda")      # seeded on the device (fast), copied below
    eng = Transformer.from_weights(args, sd, "cuda")
    eng.setup_caches(1, max_seq)
    sd = {k: v.cpu() for k, v in sd.items()}
    orc = OracleModel(args, sd)
    del sd
    orc.setup_caches(eng.max_seq_length)
    log(f"{name}: engine + oracle built in {time.time() - t0:.1f} s")
    return args, eng, orc


@pytest.fixture(scope="module")
def full(dev):
    args, eng, orc = _build(FULL, seed=0, max_seq=8200)
    yield args, eng, orc
    eng.close()


@pytest.fixture(scope="module")
def one_layer(dev):
    args, eng, orc = _build(L1, seed=0, max_seq=1024)
    yield args, eng, orc
    eng.close()


def _prefill_both(eng, orc, n, seed):
    """Seeded uniform prompt of n + 1 ids; the engine prefills the first n (slots 0..n-1) and the
    oracle's cache receives the same K/V rows. Returns the prompt (CPU int32)."""
    from flint_amd.generate import prefill
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, eng.config.vocab_size, (n + 1,), generator=g, dtype=torch.int32)
    prefill(eng, prompt[:n].to(eng.device), 0)
    eng.check()
    orc.k_cache[:, :, :n] = eng.k_cache[:, :, :n].cpu()
    orc.v_cache[:, :, :n] = eng.v_cache[:, :, :n].cpu()
    return prompt


def _check_step(label, name, eng_logits, ref, alt):
    st, fl = logit_stats(eng_logits, ref), logit_stats(alt, ref)
    bar, mbar = row_bars(name, fl)
    am_e, am_o = int(torch.argmax(eng_logits)), int(torch.argmax(ref))
    margin = top2_margin(ref)
    say(f"{label}: kernel max|d|={st['max']:.4f} mean|d|={st['mean']:.2e} within 2e-2 {st['within']:.2%} | "
        f"oracle 2nd order max|d|={fl['max']:.4f} mean|d|={fl['mean']:.2e} within {fl['within']:.2%} | "
        f"argmax {am_e}/{am_o} margin {margin:.4f}")
    assert st["max"] <= bar and st["mean"] <= mbar, (label, st, bar, mbar)
    tie = am_e != am_o
    if tie:
        assert near_tie(ref, bar), (label, am_e, am_o, margin)
    return st, fl, tie


# ------------------------------------------------------------------ config 0: one 3B layer

def test_config0_hidden_input_ctx128(one_layer):
    """one layer of the 3B model, KV slots 0..127 bf16 N(0,1), input
    activation h bf16 N(0,1) at pos 128 (129 keys), through fl_decode_hidden (the reference
    decode_mega_launch takes h). Logits within one layer's bars and >= 99.9% within 2e-2; the
    final residual written back into h: >= 99% of elements within two bf16 ulps of their own
    magnitude, and every element within two ulps of the vector's largest (an element where the
    down projection and the residual nearly cancel keeps the absolute error of the larger)."""
    args, eng, orc = one_layer
    pos = 128
    g = torch.Generator().manual_seed(100)
    k = torch.randn(1, args.n_local_heads, pos, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(1, args.n_local_heads, pos, 64, generator=g).to(torch.bfloat16)
    eng.k_cache[:, :, :pos] = k.cuda()
    eng.v_cache[:, :, :pos] = v.cuda()
    orc.k_cache[:, :, :pos] = k
    orc.v_cache[:, :, :pos] = v
    h0 = torch.randn(args.dim, generator=g).to(torch.bfloat16)
    h = h0.cuda()
    logits = torch.empty(args.vocab_size, dtype=torch.float32, device="cuda")
    tok = torch.empty(1, dtype=torch.int32, device="cuda")
    eng.decode_hidden(h, pos, token_out=tok, logits=logits)
    eng.check()

    def run():
        lg, _ = orc.forward(None, pos, h=h0.view(1, -1))
        return lg[0].float(), orc.last_residual[0].float()
    (alt, alt_h), (ref, ref_h) = oracle_pair(orc, run)
    st, _, _ = _check_step("config0 ctx128", L1, logits.cpu(), ref, alt)
    assert st["within"] >= 0.999
    assert int(tok.item()) == int(torch.argmax(logits.cpu()))
    he = h.cpu().float()

    def ulp(t):
        return torch.pow(2.0, torch.floor(torch.log2(t.abs().clamp(min=2.0 ** -126))) - 7)
    d = (he - ref_h).abs()
    own = ulp(torch.maximum(he.abs(), ref_h.abs()))
    top = ulp(torch.maximum(he.abs().max(), ref_h.abs().max()))
    log(f"config0 final residual: {float((d == 0).float().mean()):.2%} bit-identical, "
        f"{float((d <= 2 * own).float().mean()):.3%} within 2 ulp of their magnitude, max {float((d / top).max()):.2f} "
        f"ulp of the largest (oracle 2nd order: {float(((alt_h - ref_h).abs() == 0).float().mean()):.2%} identical)")
    assert float((d <= 2 * own).float().mean()) >= 0.99
    assert bool((d <= 2 * top).all())


def test_config0_pos0_known_answer(one_layer):
    """Reference bench/megakernel_decode_test.py:59-75 at the 3B layer shape: with h0 ~ N(0,1) at
    pos 0, RoPE is the identity and attention over the single key returns V of each head's KV group
    exactly (read from the kernel's own exchange buffers), and the logits match the oracle."""
    args, eng, orc = one_layer
    g = torch.Generator().manual_seed(0)
    h0 = torch.randn(args.dim, generator=g).to(torch.bfloat16)
    h = h0.cuda()
    logits = torch.empty(args.vocab_size, dtype=torch.float32, device="cuda")
    eng.decode_hidden(h, 0, logits=logits)
    eng.check()
    act = eng.activations()
    attn = act["attn"].cpu().view(args.n_head, 64)
    vrow = eng.v_cache[0, :, 0].cpu()                       # [NKV, 64], written by this launch
    rep = args.n_head // args.n_local_heads
    assert torch.equal(attn, vrow.repeat_interleave(rep, dim=0))
    # K at pos 0 is the un-rotated projection: the qkv words' k heads equal the cache row
    qkv = act["qkv"].cpu().view(-1, 64)
    assert torch.equal(qkv[args.n_head:args.n_head + args.n_local_heads], eng.k_cache[0, :, 0].cpu())

    def run():
        return orc.forward(None, 0, h=h0.view(1, -1))[0][0].float()
    alt, ref = oracle_pair(orc, run)
    st, _, _ = _check_step("config0 pos0", L1, logits.cpu(), ref, alt)
    assert st["within"] >= 0.999


# ------------------------------------------------------------------ config 2: 40 layers, ctx 512

def _flip_slack(a, b):
    """Slack of a comparison of two flip counts over the same steps: about two standard deviations
    of the difference of two binomial counts with the same rate (var ~ a + b), plus one."""
    return int(math.ceil(2.0 * math.sqrt(a + b))) + 1


def test_config2_full_model_greedy_64(full):
    """BASELINE config 2 / the north star's parity clause: the 40-layer int4 model, 512-token
    prompt, 64 greedy steps. Every step's logits within the 40-layer bars, the greedy token equal
    to the oracle's argmax on the engine's own prefix (teacher forcing) except at near-ties, and
    the kernel's mean distance over the steps no more than twice the oracle's own second-order
    distance on the same steps.

    Argmax flips are counted against the oracle's own: on every step the oracle also runs in its
    three other valid implementations (per-group summation order; exp2-based softmax / SiLU; both),
    and each implementation's flips against the default are counted on the same steps. The kernel
    may flip no more often than the worst of them plus _flip_slack. (At 40 layers the oracle's own
    implementations disagree on the greedy token at some of these steps, so "identical argmax over
    64 free-running steps" holds for no implementation; the count is what can be compared.)"""
    args, eng, orc = full
    n = 511
    prompt = _prefill_both(eng, orc, n, seed=512)
    steps = 64
    dev = eng.device
    seq = torch.empty(steps + 1, dtype=torch.int32, device=dev)
    seq[0] = int(prompt[n])
    logits = torch.empty(steps, args.vocab_size, dtype=torch.float32, device=dev)
    for i in range(steps):
        eng.decode_step(seq[i:i + 1], n + i, token_out=seq[i + 1:i + 2], logits=logits[i])
    eng.check()
    toks, lg = seq.cpu(), logits.cpu()
    ties, k_mean, o_mean, within = 0, [], [], []
    others = ("g128", "exp2")
    flips = {"g128+exp2": 0, **{o: 0 for o in others}}
    for i in range(steps):
        t = torch.tensor([int(toks[i])])
        run = lambda: orc.forward(t, n + i)[0][0].float()    # noqa: E731
        extra = {}
        for o in others:       # run before the default: each forward rewrites its cache rows
            orc.set_order(o)
            try:
                extra[o] = run()
            finally:
                orc.set_order("torch")
        alt, ref = oracle_pair(orc, run)
        st, fl, tie = _check_step(f"config2 step {i} pos {n + i}", FULL, lg[i], ref, alt)
        assert int(torch.argmax(lg[i])) == int(toks[i + 1])     # fused argmax = argmax of the logits
        am = int(torch.argmax(ref))
        fo = {"g128+exp2": int(torch.argmax(alt)) != am, **{o: int(torch.argmax(extra[o])) != am for o in others}}
        for k, v in fo.items():
            flips[k] += v
        record(f"config2 step {i:2d} pos {n + i}: margin {top2_margin(ref):.4f} kernel max|d| {st['max']:.4f} "
               f"mean {st['mean']:.2e} {'FLIP' if tie else 'same'} | oracle "
               + " ".join(f"{k} {'FLIP' if v else 'same'}" for k, v in fo.items()))
        ties += tie
        k_mean.append(st["mean"])
        o_mean.append(fl["mean"])
        within.append(st["within"])
    km, om_ = sum(k_mean) / steps, sum(o_mean) / steps
    worst = max(flips.values())
    slack = _flip_slack(ties, worst)
    record(f"config2: {steps} teacher-forced steps: kernel argmax flips {ties} (all near-ties); the oracle's "
           f"own implementations against its default: {flips}; bar {worst} + {slack}; mean|d| kernel "
           f"{km:.3e} vs oracle 2nd order {om_:.3e}, within 2e-2 {sum(within) / steps:.2%} on average")
    assert km <= 2 * om_
    assert ties <= worst + slack, (ties, flips, slack)


# ------------------------------------------------------------------ every layer, teacher-forced

def _layer_engine(eng, l, holder):
    """Layer l of eng's packed model as a one-layer engine (views of the same device tensors, no
    copy); holder keeps one Transformer whose state and KV cache are reused for every layer."""
    from flint_amd.model import PackedModel, Transformer
    pk = eng.packed
    t = {n: getattr(pk, n)[l:l + 1] for n in ("wqkv_q", "wqkv_sz", "wo_q", "wo_sz", "wgu_q", "wgu_sz",
                                              "wd_q", "wd_sz", "attn_norm", "ffn_norm")}
    t["final_norm"], t["embed"] = pk.final_norm, pk.embed
    args1 = ModelArgs.from_name(L1)
    p1 = PackedModel.from_tensors(args1, t, eng.device)
    if "e" not in holder:
        holder["e"] = Transformer(args1, p1)
        holder["e"].setup_caches(1, eng.max_seq_length)
    e1 = holder["e"]
    e1.packed, e1._cw = p1, p1.c_weights()
    return e1


def _stages(orc, l, x, n, ker, impl, slip=False):
    """The oracle's values of layer l's stages at cache position n, each stage computed from the
    kernel's own input to that stage (so a difference is that stage's, not one carried in from an
    earlier stage: a 1-ulp flip in 1% of the attention output already moves about 30% of the SwiGLU
    outputs by an ulp through the O projection, the norm and the gate/up sums):
      attn: attention with the kernel's q over the cache rows [0, n) and the kernel's new k / v row;
      act:  h1 = x + O(kernel attention), norm, gate / up, SwiGLU;
      out:  h1 (as above) + down(kernel SwiGLU output).
    impl is one of the oracle's implementations (oracle.model.IMPLS); slip plants ONE rounding
    mistake (test-only): the SwiGLU product formed in fp32 and rounded once instead of
    bf16(bf16(silu(g)) * u) (engine/model.py:227-228)."""
    import torch.nn.functional as F
    from oracle.model import IMPLS, attention, rms_norm
    lin, softmax, silu = IMPLS[impl]
    a, w = orc.args, orc.w[l]
    NH, NKV = a.n_head, a.n_local_heads
    kc = torch.cat([orc.k_cache[l, :, :n], ker["k"].view(NKV, 1, 64)], dim=1)
    vc = torch.cat([orc.v_cache[l, :, :n], ker["v"].view(NKV, 1, 64)], dim=1)
    attn = attention(ker["q"].view(NH, 64), kc, vc, torch.ones(n + 1, dtype=torch.bool), a.attn_scale,
                     softmax).view(1, -1)
    h1 = x + lin(ker["attn"].view(1, -1), w["wo"]) * a.residual_multiplier
    hn = rms_norm(h1, w["ffn_norm"], a.norm_eps)
    g, u = lin(hn, w["w1"]), lin(hn, w["w3"])
    act = (F.silu(g.float()) * u.float()).to(torch.bfloat16) if slip else silu(g) * u
    out = h1 + lin(ker["act"].view(1, -1), w["w2"]) * a.residual_multiplier
    return {"attn": attn, "act": act, "out": out}


# Bars of one layer's stage outputs against the oracle's on the same stage inputs: the fraction
# not bit-identical at most three times the oracle's second implementation's (per-group summation
# order, exp2-based softmax / SiLU) on the same inputs plus 0.3% or four values, whichever is more
# (v_dot2_f32_bf16's rare misrounding, the hardware exp2 / rcp; k and v have only 512 values), at
# least 99.5% within one ulp of their own magnitude, and every value within two ulps of the
# vector's largest. The whole layer from the same input (every stage's differences carried
# through) is logged beside the oracle's second implementation, not held to a bar: where the layer's
# update outweighs its input (layer 0, whose input is the N(0, 0.02) embedding), one flipped
# attention value moves a third of the outputs by an ulp, in either implementation.
MISMATCH_X, MISMATCH_ABS, MISMATCH_MIN_VALUES, IN1_MIN, TOP_MAX = 3.0, 3e-3, 4, 0.995, 2.0


def _per_layer(full, n, seed, label):
    """Teacher-forced check of every layer at cache position n: the oracle runs the whole model
    (recording each layer's input and values); each layer of the engine then runs alone from the
    oracle's input to that layer, over the same cache rows, through fl_decode_hidden, and each of
    its stages (q, k, v after RoPE; attention; O + residual + norm + gate/up + SwiGLU; down +
    residual) is compared with the oracle's stage on the kernel's own inputs to it. The reference
    checks its attention and MLP blocks in isolation the same way (bench/megakernel_attn_test.py:
    64-67, bench/megakernel_test.py:52-55)."""
    args, eng, orc = full
    prompt = _prefill_both(eng, orc, n, seed=seed)
    tok = torch.tensor([int(prompt[n])])
    orc.trace = []
    try:
        orc.forward(tok, n)
        ref_tr = orc.trace
    finally:
        orc.trace = None
    NH, NKV = args.n_head, args.n_local_heads
    holder, worst, fails = {}, {}, []
    slip_caught = 0
    try:
        for l in range(args.n_layer):
            e1 = _layer_engine(eng, l, holder)
            e1.k_cache[0, :, :n] = eng.k_cache[l, :, :n]
            e1.v_cache[0, :, :n] = eng.v_cache[l, :, :n]
            x = ref_tr[l]["x"]
            h = x.reshape(-1).to(eng.device).clone()
            e1.decode_hidden(h, n)
            e1.check()
            act = e1.activations()
            qkv = act["qkv"].cpu()
            ker = {"q": qkv[:NH * 64], "k": qkv[NH * 64:(NH + NKV) * 64], "v": qkv[(NH + NKV) * 64:],
                   "attn": act["attn"].cpu(), "act": act["act"].cpu(), "out": h.cpu()}
            assert torch.equal(ker["k"].view(NKV, 64), e1.k_cache[0, :, n].cpu())
            assert torch.equal(ker["v"].view(NKV, 64), e1.v_cache[0, :, n].cpu())
            # stage A (q, k, v) from the layer input: the oracle's own run, and its second
            # implementation on the same input
            orc.set_order("g128+exp2")
            orc.trace = []
            try:
                orc.layer(l, x, n)
                alt_a = orc.trace[0]
            finally:
                orc.trace = None
                orc.set_order("torch")
            ref = {k: ref_tr[l][k] for k in ("q", "k", "v")}
            alt = {k: alt_a[k] for k in ("q", "k", "v")}
            ref.update(_stages(orc, l, x, n, ker, "torch"))
            alt.update(_stages(orc, l, x, n, ker, "g128+exp2"))
            slip = _stages(orc, l, x, n, ker, "torch", slip=True)["act"]
            line = f"{label} layer {l:2d}:"
            for name in ("q", "k", "v", "attn", "act", "out"):
                sk, sa = ulp_stats(ker[name], ref[name]), ulp_stats(alt[name], ref[name])
                bar = MISMATCH_X * (1 - sa["same"]) + max(MISMATCH_ABS, MISMATCH_MIN_VALUES / ker[name].numel())
                line += (f" {name} {1 - sk['same']:.2%}/{1 - sa['same']:.2%}(bar {bar:.2%}) in1 {sk['in1']:.2%}"
                         f" top {sk['top']:.1f}")
                w = worst.setdefault(name, [0.0, 0.0, 1.0, 0.0])
                w[0] = max(w[0], 1 - sk["same"])
                w[1] = max(w[1], 1 - sa["same"])
                w[2] = min(w[2], sk["in1"])
                w[3] = max(w[3], sk["top"])
                if not (1 - sk["same"] <= bar and sk["in1"] >= IN1_MIN and sk["top"] <= TOP_MAX):
                    fails.append((l, name, sk, sa))
                if name == "act":
                    ss = ulp_stats(slip, ref["act"])
                    slip_caught += (1 - ss["same"]) > bar
                    line += f" [planted slip {1 - ss['same']:.2%}]"
            # the whole layer from the same input, differences of every stage carried through
            # (logged: config 0's figures, kernel and the oracle's second implementation)
            def in2(e, r):
                d = (e.float() - r.float()).abs().reshape(-1)
                own = bf16_ulp(torch.maximum(e.float().abs(), r.float().abs()).reshape(-1))
                return float((d <= 2 * own).float().mean())
            wk, wa = ulp_stats(ker["out"], ref_tr[l]["out"]), ulp_stats(alt_a["out"], ref_tr[l]["out"])
            line += (f" | whole layer out: kernel {1 - wk['same']:.2%} differ, {in2(ker['out'], ref_tr[l]['out']):.2%}"
                     f" within 2 ulps; oracle 2nd impl {1 - wa['same']:.2%}, {in2(alt_a['out'], ref_tr[l]['out']):.2%}")
            record(line)
    finally:
        if "e" in holder:
            holder["e"].close()
    record(f"{label}: worst over {args.n_layer} layers (kernel not bit-identical / oracle 2nd impl not "
           f"bit-identical / kernel within 1 ulp / kernel max ulps of the largest): " +
           ", ".join(f"{k} {v[0]:.2%}/{v[1]:.2%}/{v[2]:.2%}/{v[3]:.1f}" for k, v in worst.items()) +
           f"; a planted SwiGLU rounding slip fails the act bar in {slip_caught} of {args.n_layer} layers")
    assert not fails, fails[:5]
    # the bars tell a misplaced rounding from order noise: the planted slip fails the act bar in
    # (nearly) every layer; where the oracle's own second implementation moves a quarter of the
    # SwiGLU outputs (its O-projection order flips an h1 value the norm and gate/up then spread),
    # the bar rises with it and the slip can hide, which happened in one layer of 40 at ctx 8188
    assert slip_caught >= args.n_layer - 2, slip_caught


def test_every_layer_teacher_forced_ctx512(full):
    """All 40 layers, one at a time, at position 511 after a 511-token prompt (config 2's context)."""
    _per_layer(full, 511, 5120, "per-layer ctx511")


def test_every_layer_teacher_forced_ctx8192(full):
    """All 40 layers, one at a time, at position 8188 after an 8188-token prompt (config 3's
    context: attention over 8189 keys, the per-head slices merged in the O phase)."""
    _per_layer(full, 8188, 81920, "per-layer ctx8188")


# ------------------------------------------------------------------ config 3: 40 layers, ctx 8192

def test_config3_full_model_ctx8192(full):
    """the 40-layer model at context 8192 (KV 40 x 8 x 64 x 8192 bf16, about a
    quarter of the step's bytes): an 8188-token prompt prefilled, then 4 greedy steps up to
    position 8191, each against the oracle."""
    args, eng, orc = full
    n = 8188
    prompt = _prefill_both(eng, orc, n, seed=8192)
    dev = eng.device
    seq = torch.empty(5, dtype=torch.int32, device=dev)
    seq[0] = int(prompt[n])
    logits = torch.empty(4, args.vocab_size, dtype=torch.float32, device=dev)
    for i in range(4):
        eng.decode_step(seq[i:i + 1], n + i, token_out=seq[i + 1:i + 2], logits=logits[i])
    eng.check()
    toks, lg = seq.cpu(), logits.cpu()
    for i in range(4):
        t = torch.tensor([int(toks[i])])
        alt, ref = oracle_pair(orc, lambda: orc.forward(t, n + i)[0][0].float())
        _check_step(f"config3 step {i} pos {n + i}", FULL, lg[i], ref, alt)


# ------------------------------------------------------------------ config 4: verify, ctx 1024

def _tree(parent):
    m = len(parent)
    depth = torch.zeros(m, dtype=torch.int32)
    amask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            amask[i, j] = 1
            j = parent[j]
        depth[i] = int(amask[i].sum()) - 1
    return depth, amask


@pytest.mark.parametrize("kind", ["chain5", "tree8"])
def test_config4_verify_ctx1024(full, kind):
    """verify of k = 4 draft tokens (M = 5, chain) and k = 7 (an 8-node tree,
    seeded parents, depth and ancestor-or-self mask as reference spec_tree.py:101-104) at context
    1024 on the 40-layer model, with seeded uniform draft ids, against the oracle's masked
    forward of the same M tokens."""
    args, eng, orc = full
    pos = 1024
    _prefill_both(eng, orc, pos, seed=1024)
    g = torch.Generator().manual_seed(4 if kind == "chain5" else 7)
    if kind == "chain5":
        m = 5
        depth = torch.arange(m, dtype=torch.int32)
        amask = torch.tril(torch.ones(m, m, dtype=torch.uint8))
    else:
        m = 8
        parent = [-1] + [int(torch.randint(0, i, (1,), generator=g)) for i in range(1, m)]
        depth, amask = _tree(parent)
        log(f"tree parents {parent} depth {depth.tolist()}")
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32)
    tout, lg, _ = eng.verify(toks.cuda(), pos, depth=depth.cuda(), amask=amask.cuda())
    eng.check()
    lg = lg.cpu()
    alt, ref = oracle_pair(orc, lambda: orc.forward(toks, pos, depth=depth, amask=amask)[0].float())
    ties = 0
    for r in range(m):
        _, _, tie = _check_step(f"config4 {kind} row {r}", FULL, lg[r], ref[r], alt[r])
        ties += tie
    assert torch.equal(tout.cpu(), torch.argmax(lg, dim=-1).int())
    log(f"config4 {kind}: {ties} argmax differences (near-ties)")


def test_config4_verify8_equals_8_decodes(full):
    """Reference bench/verify_mega_test.py:41-59 on the full model: a greedy chain of 8 tokens
    decoded one launch at a time, then verified in ONE launch at the same slots: per position the
    reference requires rel-L2 < 0.02 and the same argmax, on the real Granite weights. On this
    synthetic model the oracle differs from itself (a second valid implementation, same step) by a
    rel-L2 of about 0.04 at 40 layers, so the bar is twice that measured value; logits within the
    40-layer bar; argmax equal except at near-ties of the decode logits."""
    args, eng, orc = full
    pos = 700
    prompt = _prefill_both(eng, orc, pos, seed=700)
    dev = eng.device
    seq = torch.empty(9, dtype=torch.int32, device=dev)
    seq[0] = int(prompt[pos])
    dl = torch.empty(8, args.vocab_size, dtype=torch.float32, device=dev)
    for i in range(8):
        eng.decode_step(seq[i:i + 1], pos + i, token_out=seq[i + 1:i + 2], logits=dl[i])
    _, vl, _ = eng.verify(seq[:8].clone(), pos)
    eng.check()
    dl, vl = dl.cpu(), vl.cpu()
    bar = logit_bar(FULL)
    t0 = torch.tensor([int(seq[0])])
    alt, ref = oracle_pair(orc, lambda: orc.forward(t0, pos)[0][0].float())
    rel_floor = float((alt - ref).norm() / ref.norm())
    log(f"oracle rel-L2 between two implementations at pos {pos}: {rel_floor:.4f}")
    for i in range(8):
        rel = float((vl[i] - dl[i]).norm() / dl[i].norm())
        st = logit_stats(vl[i], dl[i])
        same = int(torch.argmax(vl[i])) == int(torch.argmax(dl[i]))
        log(f"verify vs decode pos {pos + i}: rel-L2 {rel:.4f} max|d| {st['max']:.4f} "
            f"within 2e-2 {st['within']:.2%} argmax {'same' if same else 'DIFF'} margin {top2_margin(dl[i]):.4f}")
        assert rel <= 2 * rel_floor and st["max"] <= bar
        assert same or near_tie(dl[i], bar)
