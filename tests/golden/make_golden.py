"""Writes golden vectors of the reference gpt-fast forward for a tiny configuration.

Run in the build container, where the reference checkout exists (the GPU box has none):

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's engine/model.py (torch-only: Transformer, RMSNorm, Attention with
SDPA, interleaved RoPE, Granite multipliers; reference engine/model.py:20-269), loads it with the
dequantised int4 weights this repository's synthetic generator produces (seeded, regenerated at
test time), with the q/k rows put in the reference's interleaved RoPE order
(engine/scripts/convert_hf_checkpoint.py:75-81), and records the bf16 logits and post-norm
hidden states of a 5-token prefill followed by 3 single-token decode steps. The fixture holds
inputs and outputs only (tiny_forward.pt, loadable with torch.load(weights_only=True)).
"""
import hashlib
import importlib.util
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from flint_amd.synth import ModelArgs, synth_weights  # noqa: E402
from oracle.model import hf_to_interleaved_perm  # noqa: E402
from oracle.quant import dq_linear_weight  # noqa: E402

# tiny shape with non-default Granite multipliers, so every scalar of the forward is exercised
CONFIG = dict(block_size=64, vocab_size=512, n_layer=2, n_head=4, n_local_heads=2, dim=256,
              intermediate_size=512, rope_base=10000, norm_eps=1e-5, embedding_multiplier=12.0,
              attention_multiplier=0.015625, residual_multiplier=0.22, logits_scaling=10.0)
SEED = 4
PREFILL = [17, 300, 5, 99, 511]
DECODE = [42, 7, 256]


def weights_digest(sd):
    h = hashlib.sha256()
    for k in sorted(sd):
        h.update(k.encode())
        h.update(sd[k].view(torch.int16).numpy().tobytes())
    return h.hexdigest()


def reference_state_dict(args, sd):
    """Our model-order weights -> reference module names, int4-dequantised linears, q/k rows in
    the interleaved RoPE order."""
    hd = args.head_dim
    pq = hf_to_interleaved_perm(args.n_head, hd)
    pk = hf_to_interleaved_perm(args.n_local_heads, hd)
    out = {"tok_embeddings.weight": sd["embed"], "output.weight": sd["embed"], "norm.weight": sd["norm"]}
    for l in range(args.n_layer):
        p = f"layers.{l}."
        wqkv = dq_linear_weight(sd[p + "wqkv"])
        nq, nk = args.n_head * hd, args.n_local_heads * hd
        wq, wk, wv = wqkv[:nq], wqkv[nq:nq + nk], wqkv[nq + nk:]
        out[p + "attention.wqkv.weight"] = torch.cat([wq[pq], wk[pk], wv])
        out[p + "attention.wo.weight"] = dq_linear_weight(sd[p + "wo"])
        out[p + "feed_forward.w1.weight"] = dq_linear_weight(sd[p + "w1"])
        out[p + "feed_forward.w3.weight"] = dq_linear_weight(sd[p + "w3"])
        out[p + "feed_forward.w2.weight"] = dq_linear_weight(sd[p + "w2"])
        out[p + "attention_norm.weight"] = sd[p + "attn_norm"]
        out[p + "ffn_norm.weight"] = sd[p + "ffn_norm"]
    return out


def main(ref_root="/root/reference"):
    spec = importlib.util.spec_from_file_location("reference_model",
                                                  os.path.join(ref_root, "engine", "model.py"))
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)

    args = ModelArgs(**CONFIG)
    sd = synth_weights(args, seed=SEED)
    rargs = ref.ModelArgs(**CONFIG)
    model = ref.Transformer(rargs)
    missing, unexpected = model.load_state_dict(reference_state_dict(args, sd), strict=False)
    assert not unexpected and not [k for k in missing if "kv_cache" not in k], (missing, unexpected)
    model = model.to(torch.bfloat16).eval()
    model.setup_caches(1, CONFIG["block_size"])

    steps = []
    with torch.no_grad():
        idx = torch.tensor([PREFILL])
        pos = torch.arange(len(PREFILL))
        lg, hid = model(idx, pos, return_hidden=True)
        steps.append(dict(tokens=idx[0].clone(), pos=0, logits=lg[0].clone(), hidden=hid[0].clone()))
        p = len(PREFILL)
        for t in DECODE:
            lg, hid = model(torch.tensor([[t]]), torch.tensor([p]), return_hidden=True)
            steps.append(dict(tokens=torch.tensor([t]), pos=p, logits=lg[0].clone(), hidden=hid[0].clone()))
            p += 1
    fixture = dict(config=CONFIG, seed=SEED, weights_sha256=weights_digest(sd), steps=steps,
                   source="reference engine/model.py Transformer.forward (CPU, bf16)")
    path = os.path.join(HERE, "tiny_forward.pt")
    torch.save(fixture, path)
    print(f"wrote {path}: {len(steps)} calls, logits {tuple(steps[0]['logits'].shape)}")


if __name__ == "__main__":
    main(*sys.argv[1:])
