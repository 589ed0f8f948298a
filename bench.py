#!/usr/bin/env python3
"""Batch-1 int4 greedy decode benchmark on one MI355X: prompt 512, then timed greedy decode.

One "step" = one decoded token = ONE persistent cooperative kernel launch (fl_decode_step) over
the 40-layer 3B-class synthetic int4 model: all layers, final norm, tied bf16 LM head, greedy
argmax. Tokens chain on the device (step i reads the token step i-1 wrote), so the timed loop
has no host synchronisation. Weights are seeded random (no checkpoint exists); the prompt is
512 seeded-uniform token ids prefilled before timing (through the verify kernel, 16 tokens per
launch). After the timed decode, the speculative-verify latency (k = 4, 7 draft tokens at
context 1024) is measured beside the decode latency at the same context.

Prints ONE JSON line (the driver's contract) with `roofline` (HBM-bound: algorithmic bytes per
step / measured step time vs 8 TB/s) and `cpu_baseline` (the reference int4 decode path on the
host CPU, a bounded sample of the same workload).
"""
import argparse
import json
import os
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
METRIC = "batch-1 decode tok/s + achieved HBM GB/s (MBU) at ctx 512, 1\u00d7MI355X"
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "k_decode_traffic_flint3b_ctx512.txt")


def measured_traffic(config, ctx):
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE per dispatch, scaled by the copy-kernel calibration), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            vals = dict(line.split(":", 1) for line in f if ":" in line)
        if vals.get("config", "").strip() != f"{config} ctx {ctx}":
            return None
        return int(float(vals["traffic_bytes_per_launch"]))
    except (OSError, KeyError, ValueError):
        return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def step_bytes(args, packed, T):
    """Algorithmic HBM bytes of one decode step attending to T keys."""
    D, NL, NKV, hd = args.dim, args.n_layer, args.n_local_heads, args.head_dim
    int4 = packed.nbytes_int4()                      # packed weights + scale/zero words
    lm = args.vocab_size * D * 2                     # tied bf16 LM head
    norms = (2 * NL + 1) * D * 2
    emb_row = D * 2
    kv_read = T * NL * NKV * hd * 2 * 2              # K and V of T keys
    kv_write = NL * NKV * hd * 2 * 2
    return int4 + lm + norms + emb_row + kv_read + kv_write


def cpu_baseline(args, sd, prompt, steps):
    """The reference int4 decode path on the host CPU (oracle/cpu_int4.py, torch's CPU int4
    kernel; test infrastructure, timed here as the baseline): the same prompt prefilled (untimed),
    then `steps` greedy decode steps timed."""
    from oracle.cpu_int4 import CpuInt4Decoder
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    log(f"cpu baseline: packing int4 weights for the CPU kernel ({ncores} threads)")
    dec = CpuInt4Decoder(args, sd)
    ctx = prompt.numel()
    dec.setup_caches(ctx + steps + 8)
    t0 = time.perf_counter()
    tok = dec.prefill(prompt.cpu(), 0)
    log(f"cpu baseline: prefill of {ctx} tokens took {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    for i in range(steps):
        tok = dec.step(tok, ctx + i)
    dt = time.perf_counter() - t0
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": ncores, "kind": "port",
            "sample": f"{steps} greedy int4 decode steps at ctx {ctx}..{ctx + steps - 1} after a "
                      f"{ctx}-token prefill of the same prompt, same 40-layer model, int4 linears "
                      f"via aten::_weight_int4pack_mm_for_cpu; {model}"}


def verify_latency(model, args, dev, ctx=1024, reps=20):
    """Accept-agnostic latency of one speculative verify pass over M = k+1
    tokens (k = 4, 7; chain mask) at context `ctx`, beside the M = 1 decode step latency at the
    same context. The cache prefix is synthetic (random bf16 rows): the timing depends only on
    its length."""
    need = ctx + 32
    if model.max_seq_length < need:
        model.setup_caches(1, need)
    g = torch.Generator(device=dev).manual_seed(77)
    model.k_cache[:, :, :ctx].normal_(generator=g)
    model.v_cache[:, :, :ctx].normal_(generator=g)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / reps

    tok = torch.randint(0, args.vocab_size, (16,), device=dev, dtype=torch.int32, generator=g)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    dec_us = timed(lambda: model.decode_step(tok[:1], ctx, token_out=out))
    res = {}
    gt = torch.Generator().manual_seed(7)
    parent = [-1] + [int(torch.randint(0, i, (1,), generator=gt)) for i in range(1, 8)]
    tdepth, tmask = tree_mask(parent)
    shapes = [("5", 5, None, None), ("8", 8, None, None),
              ("tree8", 8, tdepth.to(dev), tmask.to(dev))]
    for name, m, depth, amask in shapes:
        logits = torch.empty(m, args.vocab_size, dtype=torch.float32, device=dev)
        feat = torch.empty(m, args.dim, dtype=torch.bfloat16, device=dev)
        touts = torch.empty(m, dtype=torch.int32, device=dev)
        if depth is None:
            depth = torch.arange(m, dtype=torch.int32, device=dev)
            amask = torch.tril(torch.ones(m, m, dtype=torch.uint8, device=dev))
        res[name] = round(timed(lambda: model.verify(tok[:m], ctx, depth=depth, amask=amask,
                                                     logits=logits, feat=feat,
                                                     tokens_out=touts)), 1)
    model.check()
    return {"ctx": ctx, "decode_us": round(dec_us, 1), "verify_us": res,
            "tree8_parents": parent,
            "cost_vs_decode": {k: round(v / dec_us, 3) for k, v in res.items()}}


def tree_mask(parent):
    """depth and ancestor-or-self mask of a draft tree given by parent indices (parent[0] = -1),
    as reference spec_tree.py:101-104 builds them."""
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


def handoff_probe(dev, words=2560, rounds=2000):
    """Latency of one inter-workgroup hand-off of a `words`-word tagged vector (10 KB at D = 2560
    32-bit words, an activation vector of the decode kernel), from fl_probe_handoff: one
    workgroup per CU, `rounds` chained all-to-all hand-offs; median over the workgroups of their
    time per round. Modes: across all workgroups (every XCD) over the decode kernel's uncached
    exchange memory; within each XCD's 32 workgroups over the same memory; within each XCD over
    ordinary device memory (L2-local coherent loads) -- these three poll single words with a sleep
    between polls; then across all workgroups polled as the decode kernel's waits poll (16-byte
    groups, the missing ones re-requested together, no sleep), with one round of requests in
    flight and with two (the second round 512 cycles after the first), and within each XCD polled
    that way. Also reports whether every workgroup ran on XCD blockIdx % 8 (the mapping the
    XCD-local modes assume)."""
    from flint_amd import _lib
    import ctypes
    res = {"words": words, "rounds": rounds}
    grid = ctypes.c_int32()
    for mode, name in ((0, "all_uncached_us"), (1, "xcd_uncached_us"), (2, "xcd_l2_us"),
                       (3 | 1 << 8, "all_groups_us"), (3 | 2 << 8 | 8 << 16, "all_groups_depth2_us"),
                       (4, "xcd_groups_us")):
        out = torch.zeros(2 * 1024, dtype=torch.int64, device=dev)
        for _ in range(2):      # the first call allocates and warms up
            _lib.call("fl_probe_handoff", mode, words, rounds, _lib.ptr(out), ctypes.byref(grid),
                      _lib.stream_ptr())
            torch.cuda.synchronize()
        o = out[:2 * grid.value].view(-1, 2).cpu()
        ticks = o[:, 0].double()
        info = o[:, 1]
        timeouts = int(((info >> 32) & 1).sum())
        # 100 MHz ticks: 0.01 us each
        res[name] = round(float(ticks.median()) * 0.01 / rounds, 3) if timeouts == 0 else None
        res[name.replace("_us", "_max_us")] = round(float(ticks.max()) * 0.01 / rounds, 3)
        if timeouts:
            res[name.replace("_us", "_timeouts")] = timeouts
        if mode == 0:
            xcc = (info & 0xF).tolist()
            res["xcd_is_blockidx_mod_8"] = all(x == i % 8 for i, x in enumerate(xcc))
    return res


def dequant_rate(dev, iters=2000):
    """Compute rate of the exact dequantisation with every weight already in registers
    (fl_probe_dequant), in weights per second over the slowest workgroup, beside the rate at which
    HBM delivers int4 weights with their scale/zero words (8 TB/s / 0.53125 B per weight). With an
    M = 8 MFMA product: the row layout on the vector ALUs (the verify tiles' former product), the
    tiled layout on 4x4x4 MFMAs two tiles at a time and batched over a unit's 8 tiles (the verify
    tiles' and fl_gemv_int4_tiled's unit_mma_t); with an M = 1 dot on the vector ALUs (the decode
    kernel's form): dq32 and the lane-local 4x4x4-MFMA dq32_mx."""
    from flint_amd import _lib
    import ctypes
    grid = ctypes.c_int32()
    res = {"hbm_tweights_s": round(HBM_PEAK_GBS * 1e9 / (0.5 + 4 / 128) / 1e12, 2)}
    for mode, name in ((0, "row_valu_tweights_s"), (1, "tiled_mfma_tweights_s"),
                       (2, "tiled_mfma_batched_tweights_s"), (3, "m1_row_valu_tweights_s"),
                       (4, "m1_row_mfma4_tweights_s")):
        out = torch.zeros(2 * 1024, dtype=torch.int64, device=dev)
        for _ in range(2):      # the first call loads the code object
            _lib.call("fl_probe_dequant", mode, iters, _lib.ptr(out), ctypes.byref(grid), _lib.stream_ptr())
            torch.cuda.synchronize()
        ticks = out[:2 * grid.value].view(-1, 2)[:, 0].double().cpu()
        weights = grid.value * 8 * 3 * 2048 * iters
        res[name] = round(weights / (float(ticks.max()) * 1e-8) / 1e12, 2)
    return res


def handoff_sweep(dev, rounds=2000):
    """The group-poll hand-off over its knobs (fl_probe_handoff mode 3): the sleep before each
    re-request, the number of request rounds in flight and their spacing, at 2560 and 8192 words.
    Returns {words: {label: median us per hand-off}} (python3 bench.py --handoff-sweep)."""
    from flint_amd import _lib
    import ctypes
    grid = ctypes.c_int32()

    def run(mode, words):
        out = torch.zeros(2 * 1024, dtype=torch.int64, device=dev)
        for _ in range(2):
            _lib.call("fl_probe_handoff", mode, words, rounds, _lib.ptr(out), ctypes.byref(grid),
                      _lib.stream_ptr())
            torch.cuda.synchronize()
        o = out[:2 * grid.value].view(-1, 2).cpu()
        if int(((o[:, 1] >> 32) & 1).sum()):
            return None
        return round(float(o[:, 0].double().median()) * 0.01 / rounds, 3)
    res = {}
    for words in (2560, 8192):
        r = {"single_words_sleep2": run(0, words)}
        for rs in (0, 1, 2, 4, 8, 16, 32):
            r[f"depth1_resleep{rs}"] = run(3 | 1 << 8 | rs << 24, words)
        for gap in (0, 4, 8, 12):
            r[f"depth2_gap{gap}"] = run(3 | 2 << 8 | gap << 16, words)
        for gap in (2, 6):
            r[f"depth3_gap{gap}"] = run(3 | 3 << 8 | gap << 16, words)
        res[words] = r
    return res


class KnownDraft:
    """Draft for the speculative-loop timing: proposes a known continuation `ref` of the prompt
    (chain), or that continuation hidden among two decoy siblings per level (tree: the accepted
    node is never the first child, so every pass compacts the KV cache). Once the context leaves
    `ref` it proposes nothing."""

    def __init__(self, ref, vocab, depth=5):
        self.ref, self.vocab, self.depth = ref, vocab, depth

    def _future(self, context, k):
        i = len(context)
        return self.ref[i:i + k] if context == self.ref[:i] else []

    def chain(self, context, feats, k):
        return self._future(context, k)

    def tree(self, context, feats):
        toks, pars, par = [], [], -1
        for t in self._future(context, self.depth):
            for d in ((t + 1) % self.vocab, (t + 2) % self.vocab, t):
                toks.append(int(d))
                pars.append(par)
            par = len(toks) - 1
        return toks, pars


def decode_margin(model, seq, t):
    """Top-2 logit margin of plain decode (fl_decode_step) for the token at index t of seq, given
    seq[:t] (teacher-forced: prefill seq[:t-1], one decode step of seq[t-1])."""
    from flint_amd.generate import prefill
    dev = model.device
    toks = torch.tensor(seq[:t], dtype=torch.int32, device=dev)
    if t > 1:
        prefill(model, toks[:t - 1], 0)
    lg = torch.empty(model.config.vocab_size, dtype=torch.float32, device=dev)
    model.decode_step(toks[t - 1:t], t - 1, logits=lg)
    v = torch.topk(lg, 2).values.tolist()
    return v[0] - v[1]


def spec_loop(model, args, prompt, ref, n, rounds=40):
    """Speculative greedy decoding through flint_amd.spec (one fl_verify launch per pass, plus
    fl_kv_move for a tree) at full acceptance: chain k = 4 and 7, a 16-node tree (depth 5, width
    3), and k = 0 (one verify of M = 1 per token) for the loop's own overhead. The synthetic
    model's logits are bf16-rounded and often tie at the top, and the verify kernel's fp32 sums
    depend on M, so a draft built from plain decode loses agreement at the first tie broken the
    other way; the draft is therefore re-seeded with each run's own output until a run accepts its
    whole draft (a fixed point, reached within `rounds`), and that run is the one reported.
    Wall-clock tok/s over the decode loop (prefill excluded), host loop included. Wherever a
    re-seed changed the output, the first changed token's top-2 margin under plain decode is
    recorded: a change is expected only where that margin is within the 40-layer parity bar
    (verify and decode sum in different fp32 orders); a wider margin is flagged."""
    from flint_amd.spec import SpecDecoder
    bar = 2 * 0.3671875     # twice the oracle's own implementation floor at 40 layers
    res = []
    for mode, k in (("chain", 0), ("chain", 4), ("chain", 7), ("tree", 0)):
        cur = ref
        margins = []
        for r in range(rounds):
            dec = SpecDecoder(model, KnownDraft(cur, args.vocab_size), k=k)
            out, st = dec.generate(prompt, n, mode=mode)
            if out == cur:
                break
            t = next(i for i in range(min(len(out), len(cur))) if out[i] != cur[i])
            margins.append(round(decode_margin(model, out, t), 4))
            cur = out
        model.check()
        res.append({"mode": mode, "k": k if mode == "chain" else 15, "tokens": st.tokens,
                    "passes": st.passes, "tokens_per_pass": round(st.tokens_per_pass, 2),
                    "tok_s": round(st.tokens / st.seconds, 1),
                    "ms_per_pass": round(1000 * st.seconds / max(st.passes, 1), 3),
                    "full_acceptance": out == cur, "reseeds": r,
                    "reseed_margins": margins,
                    "reseeds_beyond_bar": sum(1 for m in margins if m > bar)})
    return res


def _median_us(pairs):
    """Median over calls of the HIP-event time around each call, in us. (The mean let one host-side
    stall between an event and its launch -- once 36 ms in a sweep of 120 calls -- stand for every
    call.)"""
    t = sorted(a.elapsed_time(b) for a, b in pairs)
    return t[len(t) // 2] * 1000.0


def gemv_sweep(args, dev, sets=40, rounds=3, steady=True):
    """fl_gemv_int4 at M = 1 over the four per-layer shapes, 40 distinct weight
    sets per shape, called in layer order (QKV, O, gate/up, down of set 0, then set 1, ...) so the
    1.67 GB rotation exceeds the 256 MB Infinity Cache and every call reads its weights from HBM.
    HIP events around every call; per shape the median call time and algorithmic GB/s
    (N*K/2 int4 + N*K/128*4 scale/zero + 2K x + 2N y bytes). Weights are seeded random int4 words
    with bf16 scales 1e-3 and zeros 0 (the time does not depend on the values)."""
    from flint_amd import _lib
    D, F = args.dim, args.intermediate_size
    shapes = [("qkv", args.qkv_dim, D), ("o", D, D), ("gate_up", 2 * F, D), ("down", D, F)]
    g = torch.Generator(device=dev).manual_seed(9)
    sz_word = 0x3A83  # bf16(1e-3) scale, zero 0
    W = {}
    for name, n, k in shapes:
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (sets, n, k // 8), generator=g, device=dev, dtype=torch.int32)
        sz = torch.full((sets, n, k // 128), sz_word, dtype=torch.int32, device=dev)
        x = torch.randn(k, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty(n, dtype=torch.bfloat16, device=dev)
        W[name] = (q, sz, x, y, n, k)
    stream = torch.cuda.current_stream()
    sp = _lib.stream_ptr()

    def call(name, i):
        q, sz, x, y, n, k = W[name]
        _lib.call("fl_gemv_int4", _lib.ptr(q[i]), _lib.ptr(sz[i]), _lib.ptr(x), _lib.ptr(y), n, k, sp)
    for i in range(sets):                       # warm-up pass
        for name, _, _ in shapes:
            call(name, i)
    torch.cuda.synchronize()
    ev = {name: [] for name, _, _ in shapes}
    for _ in range(rounds):
        for i in range(sets):
            for name, _, _ in shapes:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                call(name, i)
                e1.record(stream)
                ev[name].append((e0, e1))
    torch.cuda.synchronize()
    out = {}
    for name, n, k in shapes:
        us = _median_us(ev[name])
        nbytes = n * k // 2 + n * (k // 128) * 4 + 2 * k + 2 * n
        out[name] = {"n": n, "k": k, "us": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    rot = sets * sum(W[nm][0][0].numel() * 4 + W[nm][1][0].numel() * 4 for nm, _, _ in shapes)
    # the same weights in the tiled layout, through the matrix-core GEMV (fl_gemv_int4_tiled)
    T = {}
    for name, n, k in shapes:
        q = W[name][0]
        qt = torch.empty(sets, n // 16, k // 128, 64, 4, dtype=torch.int32, device=dev)
        for i in range(sets):
            _lib.call("fl_tile_int4", _lib.ptr(q[i]), _lib.ptr(qt[i]), n, k, sp)
        T[name] = qt

    def call_t(name, i):
        q, sz, x, y, n, k = W[name]
        _lib.call("fl_gemv_int4_tiled", _lib.ptr(T[name][i]), _lib.ptr(sz[i]), _lib.ptr(x), _lib.ptr(y), n, k, sp)
    for i in range(sets):
        for name, _, _ in shapes:
            call_t(name, i)
    torch.cuda.synchronize()
    ev = {name: [] for name, _, _ in shapes}
    for _ in range(rounds):
        for i in range(sets):
            for name, _, _ in shapes:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                call_t(name, i)
                e1.record(stream)
                ev[name].append((e0, e1))
    torch.cuda.synchronize()
    tiled = {}
    for name, n, k in shapes:
        us = _median_us(ev[name])
        nbytes = n * k // 2 + n * (k // 128) * 4 + 2 * k + 2 * n
        tiled[name] = {"us": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                       "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del T
    res = {"sets_per_shape": sets, "rotation_bytes": rot, "shapes": out, "tiled_mfma": tiled}
    if steady:
        res["steady_state"] = gemv_steady(dev)
    return res


def gemv_steady(dev, reps=20):
    """Streaming rate of both M = 1 GEMVs once a call is long enough that its start-up and tail do
    not count: one N = 131072 x K = 2560 and one N = 40960 x K = 8192 matrix (about 170 MB each,
    two copies alternated so every call reads HBM), HIP events around `reps` back-to-back calls."""
    from flint_amd import _lib
    sp = _lib.stream_ptr()
    res = {}
    for n, k in ((131072, 2560), (40960, 8192)):
        g = torch.Generator(device=dev).manual_seed(3)
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (2, n, k // 8), generator=g, device=dev, dtype=torch.int32)
        sz = torch.full((2, n, k // 128), 0x3A83, dtype=torch.int32, device=dev)
        qt = torch.empty(2, n // 16, k // 128, 64, 4, dtype=torch.int32, device=dev)
        for i in range(2):
            _lib.call("fl_tile_int4", _lib.ptr(q[i]), _lib.ptr(qt[i]), n, k, sp)
        x = torch.randn(k, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty(n, dtype=torch.bfloat16, device=dev)
        nbytes = n * k // 2 + n * (k // 128) * 4
        for name, fn in (("stream", lambda i: _lib.call("fl_gemv_int4", _lib.ptr(q[i]), _lib.ptr(sz[i]), _lib.ptr(x),
                                                        _lib.ptr(y), n, k, sp)),
                         ("tiled", lambda i: _lib.call("fl_gemv_int4_tiled", _lib.ptr(qt[i]), _lib.ptr(sz[i]),
                                                       _lib.ptr(x), _lib.ptr(y), n, k, sp))):
            for i in range(4):
                fn(i % 2)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps):
                fn(i % 2)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / reps
            res[f"{name}_{n}x{k}"] = {"us": round(us, 1), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                                      "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del q, sz, qt
    return res


def long_context(model, args, dev, ctx=8192, steps=128):
    """greedy decode of `steps` tokens after a context of `ctx` keys (KV
    40 x 8 x 64 x ctx bf16, a quarter of each step's bytes). The cache prefix is synthetic (random
    bf16 rows; the step time depends only on its length); tokens chain on the device as in the
    headline loop."""
    need = ctx + steps + 8
    if model.max_seq_length < need:
        model.setup_caches(1, need)
    g = torch.Generator(device=dev).manual_seed(8192)
    model.k_cache[:, :, :ctx].normal_(generator=g)
    model.v_cache[:, :, :ctx].normal_(generator=g)
    seq = torch.empty(steps + 1, dtype=torch.int32, device=dev)
    seq[0] = 1
    for i in range(4):                                          # warm-up at the same positions
        model.decode_step(seq[i:i + 1], ctx + i, token_out=seq[i + 1:i + 2])
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        model.decode_step(seq[i:i + 1], ctx + i, token_out=seq[i + 1:i + 2])
    e1.record(stream)
    torch.cuda.synchronize()
    model.check()
    ms = e0.elapsed_time(e1) / steps
    mean_bytes = sum(step_bytes(args, model.packed, ctx + i + 1) for i in range(steps)) / steps
    gbs = mean_bytes / (ms * 1e-3) / 1e9
    return {"ctx": ctx, "steps": steps, "tok_s": round(1000.0 / ms, 1), "us_per_step": round(ms * 1000, 1),
            "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def fused_sampling(model, args, dev, pos0, steps=64):
    """Sampled decode (fl_decode_sample: temperature 0.8, top-k 200, the token drawn inside the
    decode launch) against greedy decode over the same positions, tokens chained on the device:
    time per step of each and the difference (the cost of the fused sampling)."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    seq = torch.ones(steps + 1, dtype=torch.int32, device=dev)
    res = {}
    for name in ("greedy", "sampled"):
        for rep in range(2):  # the first pass warms up
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(steps):
                if name == "greedy":
                    model.decode_step(seq[i:i + 1], pos0 + i, token_out=seq[i + 1:i + 2])
                else:
                    model.decode_sample(seq[i:i + 1], pos0 + i, 0.8, 200, seed=1, token_out=seq[i + 1:i + 2])
            e1.record(stream)
            torch.cuda.synchronize()
        res[f"{name}_us"] = round(e0.elapsed_time(e1) * 1000.0 / steps, 1)
    model.check()
    res["fused_sampling_us"] = round(res["sampled_us"] - res["greedy_us"], 1)
    return res


def sampling_latency(args, dev, reps=50):
    """fl_sample on one logit row of the model's vocabulary (temperature 0.8, top_k 200, Philox
    noise), events around `reps` back-to-back launches, beside the same with top_k off."""
    from flint_amd.generate import sample
    g = torch.Generator(device=dev).manual_seed(5)
    lg = torch.randn(args.vocab_size, device=dev, generator=g).to(torch.bfloat16).float() * 2
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    res = {}
    for name, k in (("top_k_200_us", 200), ("no_top_k_us", None)):
        for i in range(3):
            sample(lg, 0.8, k, seed=1, offset=i)
        torch.cuda.synchronize()
        e0.record()
        for i in range(reps):
            sample(lg, 0.8, k, seed=1, offset=i)
        e1.record()
        torch.cuda.synchronize()
        res[name] = round(e0.elapsed_time(e1) * 1000.0 / reps, 1)
    return res


def copy_probe(dev, mb):
    """One device-to-device copy of `mb` MiB: the known-size kernel that calibrates rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters."""
    n = mb * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: {n} bytes device-to-device")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--config", default="flint-3b")
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--spec-tokens", type=int, default=128)
    ap.add_argument("--no-long", action="store_true", help="skip config 3 (decode at ctx 8192)")
    ap.add_argument("--no-gemv", action="store_true", help="skip config 1 (HBM-cold GEMV sweep)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true",
                    help="skip the speculative-verify latency (k = 4, 7 at context 1024)")
    ap.add_argument("--no-spec", action="store_true",
                    help="skip the speculative-loop timing (chain / tree with a known draft)")
    ap.add_argument("--no-sampling", action="store_true",
                    help="skip the sampler timings (standalone and fused into the decode launch)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="run only the config-1 GEMV sweep and print its JSON (for profiling)")
    ap.add_argument("--no-steady", action="store_true",
                    help="leave the steady-state GEMV leg out of the config-1 sweep (profiling runs: its "
                         "long calls would share the sweep's kernel names and grids)")
    ap.add_argument("--handoff-sweep", action="store_true",
                    help="only the hand-off probe's group-poll sweep (fl_probe_handoff mode 3), then exit")
    ap.add_argument("--no-handoff", action="store_true",
                    help="skip the hand-off micro-benchmark (fl_probe_handoff)")
    ap.add_argument("--maps", default=None,
                    help="write the process's memory map (/proc/self/maps) to this file at the end, "
                         "to attribute the frames of a crash during interpreter exit")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="after timing, run one device-to-device copy of this many MiB (the "
                         "known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {a.gpus} is not supported (batch-1 decode "
              f"runs on a single MI355X; multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)

    from flint_amd.model import Transformer
    from flint_amd.synth import ModelArgs, synth_weights

    dev = torch.device("cuda:0")
    args = ModelArgs.from_name(a.config)
    if a.handoff_sweep:
        print(json.dumps({"handoff_sweep": handoff_sweep(dev)}), flush=True)
        return
    if a.gemv_only:
        gemv = gemv_sweep(args, dev, steady=not a.no_steady)
        log(f"config 1 (fl_gemv_int4, {gemv['rotation_bytes'] / 1e9:.2f} GB rotation): {gemv}")
        if a.copy_probe_mb > 0:
            copy_probe(dev, a.copy_probe_mb)
        print(json.dumps({"gemv_sweep": gemv}), flush=True)
        return
    log(f"synthesising {a.config} weights on the GPU")
    sd = synth_weights(args, seed=0, device=dev)
    model = Transformer.from_weights(args, sd, dev)
    torch.cuda.synchronize()
    # the cache holds the prompt and the generated tokens, as gpt-fast sizes it (generate.py:
    # max_seq_length = T + max_new_tokens); the later legs re-size it for their own contexts
    model.setup_caches(1, a.ctx + a.warmup + a.steps + 8)
    g = torch.Generator().manual_seed(1234)
    prompt = torch.randint(0, args.vocab_size, (a.ctx,), generator=g, dtype=torch.int32).to(dev)
    seq = torch.empty(a.ctx + a.warmup + a.steps, dtype=torch.int32, device=dev)
    seq[:a.ctx] = prompt
    log(f"prefill {a.ctx} tokens (verify kernel, 32 tokens per launch)")
    from flint_amd.generate import prefill
    t0 = time.perf_counter()
    prefill(model, seq[:a.ctx - 1], 0)
    torch.cuda.synchronize()
    model.check()
    log(f"prefill took {1000 * (time.perf_counter() - t0):.1f} ms")
    p0 = a.ctx - 1
    log(f"warmup {a.warmup} steps")
    for i in range(a.warmup):
        model.decode_step(seq[p0 + i:p0 + i + 1], p0 + i, token_out=seq[p0 + i + 1:p0 + i + 2])
    torch.cuda.synchronize()
    p1 = p0 + a.warmup
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log(f"timing {a.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(a.steps):
        model.decode_step(seq[p1 + i:p1 + i + 1], p1 + i, token_out=seq[p1 + i + 1:p1 + i + 2])
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    model.check()
    ms = ev0.elapsed_time(ev1) / a.steps
    tok_s = 1000.0 / ms
    mean_bytes = sum(step_bytes(args, model.packed, p1 + i + 1) for i in range(a.steps)) / a.steps
    achieved = mean_bytes / (ms * 1e-3) / 1e9
    log(f"{tok_s:.1f} tok/s, {ms * 1e3:.1f} us/step, {achieved:.0f} GB/s algorithmic "
        f"(wall {a.steps / wall:.1f} tok/s)")

    verify = None
    if not a.no_verify:
        verify = verify_latency(model, args, dev)
        log(f"verify at ctx {verify['ctx']}: decode {verify['decode_us']} us, "
            f"verify {verify['verify_us']} us")

    spec = None
    if not a.no_spec:
        n = a.spec_tokens
        # the cache holds the prompt, the n tokens and a pass's draft beyond them (at most
        # MAX_VERIFY slots)
        from flint_amd._lib import MAX_VERIFY
        need = a.ctx + n + MAX_VERIFY + 8
        if model.max_seq_length < need:
            model.setup_caches(1, need)
        # the known continuation: plain greedy decode of n tokens after the prompt
        ref = torch.empty(a.ctx + n, dtype=torch.int32, device=dev)
        ref[:a.ctx] = prompt
        from flint_amd.generate import prefill
        prefill(model, ref[:a.ctx - 1], 0)
        for i in range(n):
            model.decode_step(ref[a.ctx - 1 + i:a.ctx + i], a.ctx - 1 + i, token_out=ref[a.ctx + i:a.ctx + i + 1])
        spec = spec_loop(model, args, prompt.tolist(), ref.tolist(), n)
        for r in spec:
            log(f"spec {r['mode']} k={r['k']}: {r['tok_s']} tok/s over {r['tokens']} tokens, "
                f"{r['tokens_per_pass']} tokens per pass ({r['passes']} passes), {r['ms_per_pass']} ms "
                f"per pass (full acceptance {r['full_acceptance']} after {r['reseeds']} re-seeds, "
                f"margins {r['reseed_margins']})")

    long = None
    if not a.no_long:
        long = long_context(model, args, dev)
        log(f"config 3 (ctx {long['ctx']}): {long['tok_s']} tok/s, {long['us_per_step']} us/step, "
            f"{long['achieved_GBs']} GB/s")

    gemv = None
    if not a.no_gemv:
        gemv = gemv_sweep(args, dev, steady=not a.no_steady)
        log(f"config 1 (fl_gemv_int4, {gemv['rotation_bytes'] / 1e9:.2f} GB rotation): {gemv['shapes']}")

    sampling = None
    if not a.no_sampling:
        sampling = sampling_latency(args, dev)
        sampling.update(fused_sampling(model, args, dev, a.ctx))
        log(f"sampling over {args.vocab_size} logits: {sampling}")

    handoff = dq_rate = None
    if not a.no_handoff:
        handoff = handoff_probe(dev)
        log(f"hand-off of a {handoff['words']}-word tagged vector: {handoff}")
        dq_rate = dequant_rate(dev)
        log(f"exact dequantisation + M = 8 MFMA product, weights in registers: {dq_rate}")

    if a.copy_probe_mb > 0:
        copy_probe(dev, a.copy_probe_mb)

    cpu = None
    if not a.no_cpu_baseline:
        try:
            cpu = cpu_baseline(args, sd, prompt, a.cpu_steps)
            log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads")
        except Exception as e:  # the GPU figure stands on its own
            log(f"cpu baseline failed: {e!r}")
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random int4 weights, seeded uniform prompt ids)",
        "config": {"workload": f"{a.config}: 40-layer int4 g128 greedy decode, prompt {a.ctx}, "
                               f"{a.steps} timed tokens (BASELINE config 2)",
                   "ctx": a.ctx, "weights": "int4 groupsize 128, bf16 scale+zero; tied bf16 "
                   "LM head", "accumulate": "fp32", "global_batch": 1,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(a.config, a.ctx)},
        "cpu_baseline": cpu,
        "verify": verify,
        "spec": spec,
        "long_context": long,
        "gemv_sweep": gemv,
        "sampling": sampling,
        "handoff": handoff,
        "dequant_rate": dq_rate,
    }
    print(json.dumps(out), flush=True)
    # release the decode state (and its device memory) before interpreter shutdown
    torch.cuda.synchronize()
    model.close()
    if a.maps:
        os.makedirs(os.path.dirname(os.path.abspath(a.maps)), exist_ok=True)
        with open("/proc/self/maps") as src, open(a.maps, "w") as dst:
            dst.write(src.read())


if __name__ == "__main__":
    main()
