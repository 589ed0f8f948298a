"""Per-phase timing of the persistent decode kernel from in-kernel timestamps.

Every workgroup stamps the 100 MHz real-time clock at kernel start, when each phase's inputs
have arrived ("ready") and when its epilogue is done, then when the final norm's input has
arrived and at the end. This turns them into per-phase input wait (time spent polling for the
previous phase's tagged outputs: the synchronisation cost) and compute time, averaged over
layers, plus the step total.
"""
import ctypes

import torch

from . import _lib

TICK_US = 0.01  # 100 MHz
# per layer: P1 ready, P1 done, P2 inputs, P2 chunks, P2 merged, P2 done, P3 ready, P3 done,
#            P4 ready, P4 done, P5 ready, P5 done
PER_LAYER = 12


def slots_per_launch(n_layer):
    return 3 + PER_LAYER * n_layer


def enable(model, slots=None):
    """Attach a timestamp buffer to the model's decode state; returns (buf, grid, slots)."""
    slots = slots or slots_per_launch(model.config.n_layer)
    grid = ctypes.c_int32()
    ncu, dgrid = ctypes.c_int32(), ctypes.c_int32()
    _lib.call("fl_device_info", ctypes.byref(ncu), ctypes.byref(dgrid))
    buf = torch.zeros(max(dgrid.value, ncu.value, 1) * slots, dtype=torch.int64, device=model.device)
    _lib.call("fl_state_profile", model._state, _lib.ptr(buf), slots, ctypes.byref(grid))
    return buf, grid.value, slots


def disable(model):
    _lib.call("fl_state_profile", model._state, None, 0, None)


def analyse(buf, grid, slots, n_layer, nh=0, nkv=0):
    t = buf[: grid * slots].view(grid, slots).double().cpu() * TICK_US
    t = t - t[:, :1].min()
    L = n_layer
    lay = t[:, 1:1 + PER_LAYER * L].view(grid, L, PER_LAYER)
    prev_done = torch.cat([t[:, :1], lay[:, :-1, 11]], dim=1)         # [grid, L]
    rows = {
        "qkv+rope": (lay[..., 0] - prev_done, lay[..., 1] - lay[..., 0]),
        "attention": (lay[..., 2] - lay[..., 1], lay[..., 5] - lay[..., 2]),
        "o+resid": (lay[..., 6] - lay[..., 5], lay[..., 7] - lay[..., 6]),
        "gateup+swiglu": (lay[..., 8] - lay[..., 7], lay[..., 9] - lay[..., 8]),
        "down+resid": (lay[..., 10] - lay[..., 9], lay[..., 11] - lay[..., 10]),
    }
    att = t.new_zeros(0)
    busy = (lay[..., 5] - lay[..., 1]) > 0.5   # workgroups that ran an attention unit
    if bool(busy.any()):
        out_att = {
            "inputs_wait_us": float((lay[..., 2] - lay[..., 1])[busy].mean()),
            "chunks_us": float((lay[..., 3] - lay[..., 2])[busy].mean()),
            "merge_us": float((lay[..., 4] - lay[..., 3])[busy].mean()),
        }
    else:
        out_att = {}
    out = {"total_us": float(t[:, -1].max()), "phases": {}}
    for name, (wait, comp) in rows.items():
        d = {"compute_mean_us": float(comp.mean()), "compute_max_us": float(comp.max(0).values.mean())}
        if wait is not None:
            d["input_wait_mean_us"] = float(wait.mean())
        out["phases"][name] = d
    out["attention_units"] = out_att
    # hand-offs: when the last producer finished (relative to the median producer: imbalance) and
    # when consumers saw its outputs (relative to the last producer: exchange latency)
    prod_done = {"h->qkv": prev_done, "qkv->attention": lay[..., 1], "attn->o": lay[..., 4],
                 "h1->gateup": lay[..., 7], "act->down": lay[..., 9]}
    cons_ready = {"h->qkv": lay[..., 0], "qkv->attention": lay[..., 2], "attn->o": lay[..., 6],
                  "h1->gateup": lay[..., 8], "act->down": lay[..., 10]}
    trans = {}
    for name in prod_done:
        pd, cr = prod_done[name], cons_ready[name]
        if name == "attn->o":
            pd = torch.where(busy, pd, torch.full_like(pd, -1e30))
        if name == "qkv->attention":
            cr = torch.where(busy, cr, torch.full_like(cr, float("nan")))
        last = pd.max(0).values                                     # [L]
        med = pd.median(0).values if name != "attn->o" else last
        rel = cr - last
        trans[name] = {
            "producer_spread_us": float((last - med).mean()),
            "first_consumer_us": float(torch.nan_to_num(rel, nan=1e30).min(0).values.mean()),
            "median_consumer_us": float(rel.nanmedian(0).values.mean()),
            "last_consumer_us": float(torch.nan_to_num(rel, nan=-1e30).max(0).values.mean()),
        }
    out["handoffs"] = trans
    # per workgroup class (no attention unit / attention units by key slice: unit u of slice
    # (u / NKV) % nsl, nsl = attention workgroups / NH): how far each class's phase ends lag the
    # median workgroup's, and which class holds the last producer of each phase. A workgroup
    # ran an attention unit in most layers when its key loop took time (workgroups without a
    # unit stamp the loop's start and end back to back).
    att_wg = ((lay[..., 3] - lay[..., 2]) > 0.2).double().mean(1) > 0.5
    n_att = int(att_wg.sum())
    cls = torch.full((grid,), -1, dtype=torch.long)
    if n_att and nh and nkv and n_att % nh == 0:
        nsl = n_att // nh
        u = torch.arange(grid)
        cls = torch.where(att_wg, (u // nkv) % nsl, torch.full_like(u, -1))
    names = {-1: "no attention"}
    names.update({c: f"attention slice {c}" for c in range(int(cls.max()) + 1)})
    lag = {}
    # one class (no workgroup's key loop was stamped apart from its merge, as in the verify
    # kernel's attention by tokens) says nothing: no table then
    for pname, k in (() if int(cls.min()) == int(cls.max()) else
                     (("qkv", 1), ("attention", 5), ("o", 7), ("gateup", 9), ("down", 11))):
        end = lay[..., k]                                   # [grid, L]
        rel = end - end.median(0).values                    # lag behind the median workgroup
        last = end.argmax(0)                                # [L] the last workgroup per layer
        row = {}
        for c, nm in names.items():
            sel = cls == c
            if bool(sel.any()):
                row[nm] = {"mean_lag_us": float(rel[sel].mean()),
                           "last_share": float((cls[last] == c).double().mean())}
        lag[pname] = row
    out["class_lag"] = lag
    # critical spans: between the last workgroup to finish one phase and the last to finish the
    # next (they add up to the layer's critical path)
    ends = [prev_done.max(0).values] + [lay[..., k].max(0).values for k in (1, 5, 7, 9, 11)]
    out["spans"] = {name: float((ends[i + 1] - ends[i]).mean())
                    for i, name in enumerate(["qkv+rope", "attention", "o+resid", "gateup+swiglu",
                                              "down+resid"])}
    layer_end = lay[..., 11].max(0).values
    out["layer_critical_us"] = float((layer_end[1:] - layer_end[:-1]).mean()) if L > 1 else None
    out["final_norm_wait_us"] = float((t[:, 1 + PER_LAYER * L] - lay[:, -1, 11]).mean())
    out["lm_head_us"] = float((t[:, 2 + PER_LAYER * L] - t[:, 1 + PER_LAYER * L]).max())
    return out


def format_report(res, n_layer, label):
    """Text table of analyse()'s result (the summary kept under profiles/)."""
    out = [f"{label}: step {res['total_us']:.1f} us ({n_layer} layers; layer critical path "
           f"{res['layer_critical_us']:.2f} us; final norm wait {res['final_norm_wait_us']:.2f} us; "
           f"LM head {res['lm_head_us']:.2f} us)", "",
           f"{'phase (per layer, mean over workgroups)':42s} {'input wait us':>14s} {'compute us':>11s} "
           f"{'compute, slowest wg':>20s}"]
    for name, d in res["phases"].items():
        out.append(f"{name:42s} {d.get('input_wait_mean_us', float('nan')):14.2f} "
                   f"{d['compute_mean_us']:11.2f} {d['compute_max_us']:20.2f}")
    if res["attention_units"]:
        a = res["attention_units"]
        out += ["", f"attention workgroups: q/k/v wait {a['inputs_wait_us']:.2f} us, key loop "
                    f"{a['chunks_us']:.2f} us, wave merge {a['merge_us']:.2f} us"]
    out += ["", "critical spans (last workgroup done to last done, per layer): " +
            ", ".join(f"{k} {v:.2f} us" for k, v in res["spans"].items())]
    out += ["", f"{'hand-off (per layer)':20s} {'producer spread':>16s} {'first consumer':>15s} "
                f"{'median consumer':>16s} {'last consumer':>14s}   (us after the last producer)"]
    for name, d in res["handoffs"].items():
        out.append(f"{name:20s} {d['producer_spread_us']:16.2f} {d['first_consumer_us']:15.2f} "
                   f"{d['median_consumer_us']:16.2f} {d['last_consumer_us']:14.2f}")
    if res.get("class_lag"):
        out += ["", "phase ends by workgroup class: mean lag behind the median workgroup (us) / share of "
                    "layers in which the class holds the last workgroup"]
        for pname, row in res["class_lag"].items():
            out.append(f"  {pname:10s} " + "   ".join(f"{nm}: {d['mean_lag_us']:+.2f} / {d['last_share']:.0%}"
                                                    for nm, d in row.items()))
    return "\n".join(out)


def main(argv=None):
    """python -m flint_amd.profile [--config flint-3b] [--ctx 512] [--steps 8]: one model on the
    GPU, a ctx-token prompt prefilled, `steps` decode steps with timestamps on; prints the
    per-phase table of the last step."""
    import argparse
    from .generate import prefill
    from .model import Transformer
    from .synth import ModelArgs, synth_weights
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="flint-3b")
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--save", default=None, help="also save the raw timestamp buffer (torch.save) to this file")
    ap.add_argument("--verify", type=int, default=0,
                    help="profile fl_verify of this many chain tokens (at position ctx) instead of decode")
    a = ap.parse_args(argv)
    args = ModelArgs.from_name(a.config)
    dev = torch.device("cuda:0")
    model = Transformer.from_weights(args, synth_weights(args, 0, device=dev), dev)
    model.setup_caches(1, a.ctx + a.steps + max(a.verify, 0) + 8)
    g = torch.Generator().manual_seed(1234)
    seq = torch.empty(a.ctx + a.steps, dtype=torch.int32, device=dev)
    seq[:a.ctx] = torch.randint(0, args.vocab_size, (a.ctx,), generator=g, dtype=torch.int32).to(dev)
    prefill(model, seq[:a.ctx - 1], 0)
    buf, grid, slots = enable(model)
    if a.verify:
        toks = torch.randint(0, args.vocab_size, (a.verify,), generator=g, dtype=torch.int32).to(dev)
        for _ in range(a.steps):
            model.verify(toks, a.ctx)
        label = f"{a.config} k_verify M={a.verify} at ctx {a.ctx}, {grid} workgroups"
    else:
        for i in range(a.steps):
            p = a.ctx - 1 + i
            model.decode_step(seq[p:p + 1], p, token_out=seq[p + 1:p + 2])
        label = f"{a.config} k_decode at ctx {a.ctx + a.steps - 1}, {grid} workgroups"
    model.check()
    disable(model)
    if a.save:
        torch.save({"buf": buf.cpu(), "grid": grid, "slots": slots, "n_layer": args.n_layer,
                    "n_head": args.n_head, "n_kv": args.n_local_heads}, a.save)
    res = analyse(buf, grid, slots, args.n_layer, args.n_head, args.n_local_heads)
    print(format_report(res, args.n_layer, label))
    model.close()


if __name__ == "__main__":
    main()
