"""The torch-extension binding (flint_amd/_torch_ops, csrc/fl_torch.cpp: pybind11 ops over torch
tensors, the form of the reference's decode_mega_launch / verify_mega_launch) against the ctypes
path over the same C ABI: the same launches, so bit-identical logits, tokens, features and
written-back residuals."""
import pytest
import torch

from tests.helpers import fill_kv_random, make_pair

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def both(dev):
    import flint_amd._torch_ops as ops
    args, sd, eng, orc = make_pair("small", seed=4, weight_device="cuda")
    eng.setup_caches(1, 512)
    orc.setup_caches(eng.max_seq_length)
    pk = eng.packed
    kc, vc = torch.zeros_like(eng.k_cache), torch.zeros_like(eng.v_cache)
    ext = ops.Engine(pk.wqkv_q, pk.wqkv_sz, pk.wo_q, pk.wo_sz, pk.wgu_q, pk.wgu_sz, pk.wd_q, pk.wd_sz,
                     pk.attn_norm, pk.ffn_norm, pk.final_norm, pk.embed, pk.rope, kc, vc,
                     args.norm_eps, args.embedding_multiplier, args.attn_scale,
                     args.residual_multiplier, args.logits_scaling)
    yield args, eng, orc, ext, kc, vc, ops
    del ext
    eng.close()


def _sync_cache(eng, orc, kc, vc, pos):
    fill_kv_random(eng, orc, pos, seed=pos + 3)
    kc.copy_(eng.k_cache)
    vc.copy_(eng.v_cache)


def test_ext_decode_step_and_hidden(both):
    args, eng, orc, ext, kc, vc, ops = both
    s = torch.cuda.current_stream().cuda_stream
    pos = 100
    _sync_cache(eng, orc, kc, vc, pos)
    tok = torch.tensor([17], dtype=torch.int32, device="cuda")
    t_ext, lg_ext = ext.decode_step(tok, pos, s)
    ext.check(s)
    lg = torch.empty(args.vocab_size, dtype=torch.float32, device="cuda")
    t_c = eng.decode_step(tok, pos, token_out=torch.empty(1, dtype=torch.int32, device="cuda"), logits=lg)
    eng.check()
    assert int(t_ext.item()) == int(t_c.item())
    assert torch.equal(lg_ext, lg)
    assert torch.equal(kc[:, :, pos], eng.k_cache[:, :, pos])
    # the reference's h form: h is mutated in place into the final residual
    g = torch.Generator(device="cuda").manual_seed(1)
    h0 = torch.randn(args.dim, device="cuda", generator=g).to(torch.bfloat16)
    h1, h2 = h0.clone(), h0.clone()
    lg_ext = ext.decode_hidden(h1, pos + 1, s)
    eng.decode_hidden(h2, pos + 1, logits=lg)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(lg_ext, lg) and not torch.equal(h1, h0)
    with pytest.raises(RuntimeError, match="h"):
        ext.decode_hidden(h1[:-1], pos, s)


def test_ext_verify_and_linear(both):
    args, eng, orc, ext, kc, vc, ops = both
    s = torch.cuda.current_stream().cuda_stream
    pos, m = 200, 6
    _sync_cache(eng, orc, kc, vc, pos)
    toks = torch.arange(3, 3 + m, dtype=torch.int32, device="cuda")
    depth = torch.tensor([0, 1, 1, 2, 2, 3], dtype=torch.int32, device="cuda")
    parent = [-1, 0, 0, 1, 2, 3]
    amask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            amask[i, j] = 1
            j = parent[j]
    amask = amask.cuda()
    to_e, lg_e, ft_e = ext.verify(toks, depth, amask, pos, s)
    ext.check(s)
    to_c, lg_c, ft_c = eng.verify(toks, pos, depth=depth, amask=amask)
    eng.check()
    assert torch.equal(to_e, to_c) and torch.equal(lg_e, lg_c) and torch.equal(ft_e, ft_c)
    from flint_amd.quantize import WeightOnlyInt4Linear
    w = (torch.randn(768, 1280, generator=torch.Generator().manual_seed(2)) * 0.02).to(torch.bfloat16)
    lin = WeightOnlyInt4Linear.from_float(w.cuda())
    for rows in (1, 7, 32):
        x = torch.randn(rows, 1280, device="cuda").to(torch.bfloat16)
        assert torch.equal(ops.int4_linear(x, lin.weight, lin.scales_and_zeros, s), lin(x))
