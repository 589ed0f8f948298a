"""On-disk weight formats.

- HF safetensors of a Granite / Llama-style checkpoint (the files flint's chat.py:32-52
  load_packed reads): q/k/v rows stay in HF (NEOX) order, which is the order the decode kernel's
  half-split RoPE takes; the embedding doubles as the tied LM head.
- gpt-fast's bf16 `model.pth` (engine/scripts/convert_hf_checkpoint.py:57-113): its wq and wk rows
  were permuted to the interleaved RoPE order (:75-81); they are permuted back.
- gpt-fast's int4 `model_int4.g128.pth` (engine/quantize.py:436-437, 571-603) is refused: it
  holds `_convert_weight_to_int4pack` tiles, a layout private to the CUDA kernel. Quantise from
  the bf16 checkpoint instead (the same group scheme, on the GPU).
- flint_amd's own packed int4 file (save_packed / load_packed): the quantised tensors in this
  library's layout with the model's arguments, so a model is quantised once and later loads
  without the bf16 weights.

state dicts use flint_amd.synth's keys: layers.{l}.{wqkv,wo,w1,w3,w2,attn_norm,ffn_norm}, norm,
embed.
"""
import dataclasses
import glob
import json
import os

import torch

from .synth import ModelArgs

PACKED_FORMAT = "flint_amd-int4-g128"
PACKED_VERSION = "1"
PACKED_TENSORS = ("wqkv_q", "wqkv_sz", "wo_q", "wo_sz", "wgu_q", "wgu_sz", "wd_q", "wd_sz",
                  "attn_norm", "ffn_norm", "final_norm", "embed")


def _check_shapes(sd, args):
    D, F, L, V = args.dim, args.intermediate_size, args.n_layer, args.vocab_size
    want = {"norm": (D,), "embed": (V, D)}
    for l in range(L):
        p = f"layers.{l}."
        want.update({p + "wqkv": (args.qkv_dim, D), p + "wo": (D, D), p + "w1": (F, D), p + "w3": (F, D),
                     p + "w2": (D, F), p + "attn_norm": (D,), p + "ffn_norm": (D,)})
    for k, shp in want.items():
        if k not in sd:
            raise KeyError(f"checkpoint has no tensor for {k}")
        if tuple(sd[k].shape) != shp:
            raise ValueError(f"{k}: shape {tuple(sd[k].shape)}, the model arguments need {shp}")
    return sd


def _tied(embed, head, what):
    if head is not None and not torch.equal(head.to(embed.dtype), embed):
        raise ValueError(f"{what} differs from the embedding: this engine's LM head is the tied embedding")


def state_dict_from_hf(hf, args: ModelArgs):
    """HF (transformers) names -> flint_amd keys, as chat.py:38-50 maps them."""
    sd = {}
    for l in range(args.n_layer):
        p, q = f"model.layers.{l}.", f"layers.{l}."
        sd[q + "wqkv"] = torch.cat([hf[p + "self_attn.q_proj.weight"], hf[p + "self_attn.k_proj.weight"],
                                    hf[p + "self_attn.v_proj.weight"]], 0)
        sd[q + "wo"] = hf[p + "self_attn.o_proj.weight"]
        sd[q + "w1"] = hf[p + "mlp.gate_proj.weight"]
        sd[q + "w3"] = hf[p + "mlp.up_proj.weight"]
        sd[q + "w2"] = hf[p + "mlp.down_proj.weight"]
        sd[q + "attn_norm"] = hf[p + "input_layernorm.weight"]
        sd[q + "ffn_norm"] = hf[p + "post_attention_layernorm.weight"]
    sd["norm"] = hf["model.norm.weight"]
    sd["embed"] = hf["model.embed_tokens.weight"]
    _tied(sd["embed"], hf.get("lm_head.weight"), "lm_head.weight")
    return _check_shapes(sd, args)


def load_hf_safetensors(path, args: ModelArgs, device="cpu"):
    """Every *.safetensors file of a checkpoint directory (or one file) -> flint_amd state dict."""
    from safetensors.torch import load_file
    files = sorted(glob.glob(os.path.join(path, "*.safetensors"))) if os.path.isdir(path) else [path]
    if not files:
        raise FileNotFoundError(f"no .safetensors files under {path}")
    hf = {}
    for f in files:
        hf.update(load_file(f, device=str(device)))
    return state_dict_from_hf(hf, args)


def hf_to_interleaved_perm(n_heads, head_dim):
    """Row permutation from HF (NEOX half-split) order to gpt-fast's interleaved order: row
    (h, t, i) of a head (t in {0, 1}, i < head_dim / 2) goes to (h, i, t), as gpt-fast's
    convert_hf_checkpoint.py:75-81 permute does; w_interleaved = w_hf[perm]."""
    i = torch.arange(head_dim // 2)
    within = torch.stack([i, i + head_dim // 2], dim=1).reshape(-1)
    return (torch.arange(n_heads).unsqueeze(1) * head_dim + within.unsqueeze(0)).reshape(-1)


def interleaved_to_hf(w, n_head, head_dim):
    """Undo gpt-fast's permute (convert_hf_checkpoint.py:75-81), which takes HF rows (h, t, i) to
    (h, i, t) for t in {0, 1}, i < head_dim / 2."""
    dim = w.shape[-1]
    return w.view(n_head, head_dim // 2, 2, dim).transpose(1, 2).reshape(n_head * head_dim, dim)


def state_dict_from_gptfast(gf, args: ModelArgs):
    """gpt-fast bf16 names (convert_hf_checkpoint.py:57-71) -> flint_amd keys; wq / wk rows back
    to HF order."""
    if any(k.endswith("scales_and_zeros") for k in gf):
        raise NotImplementedError(
            "gpt-fast int4 checkpoints hold _convert_weight_to_int4pack tiles, a layout private to "
            "the CUDA kernel; load the bf16 model.pth and quantise it (PackedModel / save_packed)")
    hd, nh, nkv = args.head_dim, args.n_head, args.n_local_heads
    sd = {}
    for l in range(args.n_layer):
        p, q = f"layers.{l}.", f"layers.{l}."
        wqkv = gf[p + "attention.wqkv.weight"]
        wq, wk, wv = wqkv.split([nh * hd, nkv * hd, nkv * hd], 0)
        sd[q + "wqkv"] = torch.cat([interleaved_to_hf(wq, nh, hd), interleaved_to_hf(wk, nkv, hd), wv], 0)
        sd[q + "wo"] = gf[p + "attention.wo.weight"]
        sd[q + "w1"] = gf[p + "feed_forward.w1.weight"]
        sd[q + "w3"] = gf[p + "feed_forward.w3.weight"]
        sd[q + "w2"] = gf[p + "feed_forward.w2.weight"]
        sd[q + "attn_norm"] = gf[p + "attention_norm.weight"]
        sd[q + "ffn_norm"] = gf[p + "ffn_norm.weight"]
    sd["norm"] = gf["norm.weight"]
    sd["embed"] = gf["tok_embeddings.weight"]
    _tied(sd["embed"], gf.get("output.weight"), "output.weight")
    return _check_shapes(sd, args)


def load_gptfast_checkpoint(path, args: ModelArgs):
    """gpt-fast model.pth -> flint_amd state dict (torch.load with weights_only: nothing in the file
    is executed)."""
    gf = torch.load(path, map_location="cpu", mmap=True, weights_only=True)
    return state_dict_from_gptfast(gf, args)


def save_packed(packed, path):
    """The quantised model (a flint_amd.model.PackedModel) -> one safetensors file."""
    from safetensors.torch import save_file
    tensors = {n: getattr(packed, n).detach().contiguous().cpu() for n in PACKED_TENSORS}
    meta = {"format": PACKED_FORMAT, "version": PACKED_VERSION,
            "model_args": json.dumps(dataclasses.asdict(packed.args))}
    save_file(tensors, path, metadata=meta)


def load_packed(path, device="cuda"):
    """A file written by save_packed -> (ModelArgs, PackedModel) on `device`, no re-quantisation."""
    from safetensors import safe_open
    from safetensors.torch import load_file
    from .model import PackedModel
    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    if meta.get("format") != PACKED_FORMAT or meta.get("version") != PACKED_VERSION:
        raise ValueError(f"{path}: not a {PACKED_FORMAT} v{PACKED_VERSION} file ({meta.get('format')!r} "
                         f"v{meta.get('version')!r})")
    args = ModelArgs(**json.loads(meta["model_args"]))
    tensors = load_file(path, device=str(device))
    return args, PackedModel.from_tensors(args, tensors, device)
