"""On-disk weight formats (flint_amd/checkpoint.py) on the CPU: HF safetensors (the files
reference chat.py:32-52 reads) and gpt-fast's bf16 model.pth (engine/scripts/
convert_hf_checkpoint.py:57-113, whose q/k row permutation :75-81 is restated here in the forward
direction and must be undone exactly), each written from seeded weights and read back
bit-identical; gpt-fast int4 files and untied LM heads are refused."""
import pytest
import torch

from flint_amd.checkpoint import (interleaved_to_hf, load_gptfast_checkpoint, load_hf_safetensors,
                                  state_dict_from_gptfast, state_dict_from_hf)
from flint_amd.synth import ModelArgs, synth_weights
from oracle.model import hf_to_interleaved_perm
import flint_amd.checkpoint as ck


def _args():
    return ModelArgs(block_size=256, n_layer=2, n_head=8, n_local_heads=2, dim=512,
                     intermediate_size=1024, vocab_size=640)


def _hf_names(sd, args):
    hf = {}
    hd = args.head_dim
    for l in range(args.n_layer):
        p, q = f"model.layers.{l}.", f"layers.{l}."
        wq, wk, wv = sd[q + "wqkv"].split([args.n_head * hd, args.n_local_heads * hd, args.n_local_heads * hd])
        hf[p + "self_attn.q_proj.weight"] = wq.clone()
        hf[p + "self_attn.k_proj.weight"] = wk.clone()
        hf[p + "self_attn.v_proj.weight"] = wv.clone()
        hf[p + "self_attn.o_proj.weight"] = sd[q + "wo"]
        hf[p + "mlp.gate_proj.weight"] = sd[q + "w1"]
        hf[p + "mlp.up_proj.weight"] = sd[q + "w3"]
        hf[p + "mlp.down_proj.weight"] = sd[q + "w2"]
        hf[p + "input_layernorm.weight"] = sd[q + "attn_norm"]
        hf[p + "post_attention_layernorm.weight"] = sd[q + "ffn_norm"]
    hf["model.norm.weight"] = sd["norm"]
    hf["model.embed_tokens.weight"] = sd["embed"]
    return hf


def _same(a, b):
    assert set(a) == set(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), k


def test_hf_safetensors_round_trip(tmp_path):
    from safetensors.torch import save_file
    args = _args()
    sd = synth_weights(args, seed=3)
    hf = _hf_names(sd, args)
    keys = sorted(hf)
    save_file({k: hf[k].contiguous() for k in keys[: len(keys) // 2]}, str(tmp_path / "model-00001.safetensors"))
    save_file({k: hf[k].contiguous() for k in keys[len(keys) // 2:]}, str(tmp_path / "model-00002.safetensors"))
    _same(load_hf_safetensors(str(tmp_path), args), sd)
    hf2 = dict(hf, **{"lm_head.weight": hf["model.embed_tokens.weight"].clone()})
    _same(state_dict_from_hf(hf2, args), sd)            # a tied lm_head copy is accepted
    hf2["lm_head.weight"][0, 0] += 1
    with pytest.raises(ValueError):
        state_dict_from_hf(hf2, args)
    with pytest.raises(KeyError):
        state_dict_from_hf({k: v for k, v in hf.items() if "layers.1.mlp.up" not in k}, args)
    bad = dict(hf)
    bad["model.norm.weight"] = torch.ones(7, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        state_dict_from_hf(bad, args)


def _gptfast_permute(w, n_head, head_dim, dim):
    # the forward permutation of convert_hf_checkpoint.py:75-81
    return w.view(n_head, 2, head_dim // 2, dim).transpose(1, 2).reshape(head_dim * n_head, dim)


def test_interleaved_to_hf_inverts_the_permute():
    for nh, hd, dim in ((8, 64, 512), (40, 64, 2560), (2, 128, 256)):
        w = torch.randn(nh * hd, dim)
        assert torch.equal(interleaved_to_hf(_gptfast_permute(w, nh, hd, dim), nh, hd), w)
        assert torch.equal(interleaved_to_hf(w[hf_to_interleaved_perm(nh, hd)], nh, hd), w)
        # the product's forward permutation equals the reference permute (and the oracle's)
        perm = ck.hf_to_interleaved_perm(nh, hd)
        assert torch.equal(w[perm], _gptfast_permute(w, nh, hd, dim))
        assert torch.equal(perm, hf_to_interleaved_perm(nh, hd))


def _gptfast_names(sd, args):
    """gpt-fast bf16 state dict (convert_hf_checkpoint.py:57-71 names, q/k rows permuted)."""
    hd, D = args.head_dim, args.dim
    gf = {}
    for l in range(args.n_layer):
        p = f"layers.{l}."
        wq, wk, wv = sd[p + "wqkv"].split([args.n_head * hd, args.n_local_heads * hd, args.n_local_heads * hd])
        gf[p + "attention.wqkv.weight"] = torch.cat([_gptfast_permute(wq, args.n_head, hd, D),
                                                     _gptfast_permute(wk, args.n_local_heads, hd, D), wv])
        gf[p + "attention.wo.weight"] = sd[p + "wo"]
        gf[p + "feed_forward.w1.weight"] = sd[p + "w1"]
        gf[p + "feed_forward.w3.weight"] = sd[p + "w3"]
        gf[p + "feed_forward.w2.weight"] = sd[p + "w2"]
        gf[p + "attention_norm.weight"] = sd[p + "attn_norm"]
        gf[p + "ffn_norm.weight"] = sd[p + "ffn_norm"]
    gf["norm.weight"] = sd["norm"]
    gf["tok_embeddings.weight"] = sd["embed"]
    gf["output.weight"] = sd["embed"].clone()
    return gf


def test_gptfast_checkpoint_round_trip(tmp_path):
    args = _args()
    sd = synth_weights(args, seed=4)
    gf = _gptfast_names(sd, args)
    torch.save(gf, tmp_path / "model.pth")
    _same(load_gptfast_checkpoint(str(tmp_path / "model.pth"), args), sd)
    q4 = dict(gf)
    q4["layers.0.attention.wo.scales_and_zeros"] = torch.zeros(4, 512, 2, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        state_dict_from_gptfast(q4, args)
