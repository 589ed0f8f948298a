"""GPU: flint_amd's packed int4 file (save_packed / load_packed) reloads bit-identical and the
reloaded model decodes bit-identically; a model read from HF safetensors quantises to the same
int4 tensors as the in-memory weights it was written from."""
import pytest
import torch

from tests.helpers import log

pytestmark = pytest.mark.gpu


def test_packed_file_round_trip_and_decode(dev, tmp_path):
    from flint_amd.checkpoint import PACKED_TENSORS, load_packed, save_packed
    from flint_amd.model import PackedModel, Transformer
    from flint_amd.synth import ModelArgs, synth_weights
    args = ModelArgs.from_name("tiny")
    sd = synth_weights(args, seed=8)
    pk = PackedModel(args, sd, dev)
    path = str(tmp_path / "tiny.int4.safetensors")
    save_packed(pk, path)
    args2, pk2 = load_packed(path, dev)
    assert args2 == args
    for n in PACKED_TENSORS:
        assert torch.equal(getattr(pk, n), getattr(pk2, n)), n
    outs = []
    for p in (pk, pk2):
        eng = Transformer(args, p)
        eng.setup_caches(1, 64)
        lg = torch.empty(args.vocab_size, dtype=torch.float32, device=dev)
        tok = torch.tensor([5], dtype=torch.int32, device=dev)
        for pos in range(4):
            tok = eng.decode_step(tok, pos, logits=lg).clone()
        eng.check()
        outs.append(lg.clone())
        eng.close()
    assert torch.equal(outs[0], outs[1])
    log(f"packed file {path}: {sum(getattr(pk, n).numel() * getattr(pk, n).element_size() for n in PACKED_TENSORS)} bytes of tensors")


def test_hf_loaded_weights_pack_identically(dev, tmp_path):
    from safetensors.torch import save_file
    from flint_amd.checkpoint import load_hf_safetensors
    from flint_amd.model import PackedModel
    from flint_amd.synth import ModelArgs, synth_weights
    from tests.test_checkpoint import _hf_names
    args = ModelArgs.from_name("tiny")
    sd = synth_weights(args, seed=9)
    save_file({k: v.contiguous() for k, v in _hf_names(sd, args).items()}, str(tmp_path / "m.safetensors"))
    a = PackedModel(args, sd, dev)
    b = PackedModel(args, load_hf_safetensors(str(tmp_path), args), dev)
    for n in ("wqkv_q", "wqkv_sz", "wgu_q", "wgu_sz", "wd_q", "embed", "attn_norm"):
        assert torch.equal(getattr(a, n), getattr(b, n)), n


@pytest.mark.parametrize("fmt", ["hf", "gptfast", "packed"])
def test_checkpoint_loaded_model_matches_oracle(dev, tmp_path, fmt):
    """A model loaded from a file through the product's loaders (HF safetensors, gpt-fast bf16
    model.pth with its q/k permutation, flint_amd's packed int4 file) decodes like the oracle built
    from the seeded weights the file was written from: a prompt prefilled, then 8 greedy steps,
    every step's logits within the configuration's parity bars and the same argmax except at
    near-ties. A name-mapping, permutation or packing mistake in a loader shows here."""
    from safetensors.torch import save_file
    from flint_amd.checkpoint import (load_gptfast_checkpoint, load_hf_safetensors, load_packed,
                                      save_packed)
    from flint_amd.generate import prefill
    from flint_amd.model import PackedModel, Transformer
    from flint_amd.synth import ModelArgs, synth_weights
    from oracle.model import OracleModel
    from tests.helpers import compare_logits, logit_bar, near_tie
    from tests.test_checkpoint import _gptfast_names, _hf_names
    name = "small"
    args = ModelArgs.from_name(name)
    sd = synth_weights(args, seed=17)
    if fmt == "hf":
        save_file({k: v.contiguous() for k, v in _hf_names(sd, args).items()}, str(tmp_path / "m.safetensors"))
        eng = Transformer.from_weights(args, load_hf_safetensors(str(tmp_path), args), dev)
    elif fmt == "gptfast":
        torch.save(_gptfast_names(sd, args), tmp_path / "model.pth")
        eng = Transformer.from_weights(args, load_gptfast_checkpoint(str(tmp_path / "model.pth"), args), dev)
    else:
        save_packed(PackedModel(args, sd, dev), str(tmp_path / "m.int4.safetensors"))
        args2, pk = load_packed(str(tmp_path / "m.int4.safetensors"), dev)
        eng = Transformer(args2, pk)
    orc = OracleModel(args, sd)
    P, steps = 30, 8
    g = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, args.vocab_size, (P + steps,), generator=g, dtype=torch.int32)
    eng.setup_caches(1, P + steps + 8)
    orc.setup_caches(eng.max_seq_length)
    prefill(eng, prompt[:P].to(dev), 0)
    orc.forward(prompt[:P], 0)
    lg = torch.empty(args.vocab_size, dtype=torch.float32, device=dev)
    bar = logit_bar(name)
    for i in range(steps):
        t = prompt[P + i:P + i + 1]
        out = eng.decode_step(t.to(dev), P + i, logits=lg)
        lo = orc.forward(t, P + i)[0][0]
        ok, d, within, same = compare_logits(lg.cpu(), lo, name)
        log(f"{fmt} step {i}: max|dlogit|={d:.3e} ({within:.1%} within 2e-2) argmax {int(out.item())}/{int(lo.argmax())}")
        assert ok
        assert int(out.item()) == int(torch.argmax(lo.float())) or near_tie(lo, bar)
    eng.check()
    eng.close()
