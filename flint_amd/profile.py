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


def analyse(buf, grid, slots, n_layer):
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
    layer_end = lay[..., 11].max(0).values
    out["layer_critical_us"] = float((layer_end[1:] - layer_end[:-1]).mean()) if L > 1 else None
    out["final_norm_wait_us"] = float((t[:, 1 + PER_LAYER * L] - lay[:, -1, 11]).mean())
    out["lm_head_us"] = float((t[:, 2 + PER_LAYER * L] - t[:, 1 + PER_LAYER * L]).max())
    return out
