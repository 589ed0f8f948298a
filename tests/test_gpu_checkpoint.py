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
