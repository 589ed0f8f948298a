"""The cooperative launch path (FLINT_AMD_COOPERATIVE=1): decode, verify and the standalone
sampler launched with hipLaunchCooperativeKernel, as the reference launches decode_mega
(kernels/megakernel_decode.cu:235). The default is a plain launch (every workgroup of the grid
is resident at once on an idle device, and every inter-workgroup wait is bounded); the kernels
are the same either way, so both launch modes must give bit-identical outputs, and the
cooperative one must match the oracle like the default.
"""
import pytest
import torch

from tests.helpers import check_rows, fill_kv_random, log, oracle_pair

pytestmark = pytest.mark.gpu

NAME = "flint-3b-l1"


@pytest.fixture(scope="module")
def engines(dev):
    """(args, plain engine, cooperative engine, oracle) over the same packed weights and cache
    contents: the launch mode is read when a state is created."""
    from flint_amd.model import Transformer
    from flint_amd.synth import ModelArgs, synth_weights
    from oracle.model import OracleModel
    args = ModelArgs.from_name(NAME)
    sd = synth_weights(args, 11, device="cuda")
    plain = Transformer.from_weights(args, sd, "cuda")
    plain.setup_caches(1, 1024)
    mp = pytest.MonkeyPatch()
    mp.setenv("FLINT_AMD_COOPERATIVE", "1")
    try:
        coop = Transformer(args, plain.packed)
        coop.setup_caches(1, 1024)
    finally:
        mp.undo()
    orc = OracleModel(args, {k: v.cpu() for k, v in sd.items()})
    orc.setup_caches(coop.max_seq_length)
    yield args, plain, coop, orc
    coop.close()
    plain.close()


def _same_cache(plain, coop, orc, pos):
    fill_kv_random(coop, orc, pos, seed=pos)
    plain.k_cache.copy_(coop.k_cache)
    plain.v_cache.copy_(coop.v_cache)


@pytest.mark.parametrize("pos", [5, 300, 900])
def test_cooperative_decode_equals_plain_and_oracle(engines, pos):
    args, plain, coop, orc = engines
    _same_cache(plain, coop, orc, pos)
    tok = torch.tensor([(13 * pos + 1) % args.vocab_size], dtype=torch.int32, device="cuda")
    out = {}
    for name, e in (("plain", plain), ("coop", coop)):
        lg = torch.empty(args.vocab_size, dtype=torch.float32, device="cuda")
        t = e.decode_step(tok, pos, token_out=torch.empty(1, dtype=torch.int32, device="cuda"), logits=lg)
        e.check()
        out[name] = (int(t.item()), lg.cpu(), e.k_cache[0, :, pos].cpu())
    log(f"pos {pos}: plain token {out['plain'][0]}, cooperative token {out['coop'][0]}")
    assert out["plain"][0] == out["coop"][0]
    assert torch.equal(out["plain"][1], out["coop"][1])
    assert torch.equal(out["plain"][2], out["coop"][2])
    alt, ref = oracle_pair(orc, lambda: orc.forward(tok.cpu(), pos)[0].float())
    check_rows(out["coop"][1].view(1, -1), ref, alt, NAME, f"cooperative decode pos {pos}")


@pytest.mark.parametrize("m", [5, 8])
def test_cooperative_verify_equals_plain_and_oracle(engines, m):
    args, plain, coop, orc = engines
    pos = 500
    _same_cache(plain, coop, orc, pos)
    g = torch.Generator().manual_seed(m)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32)
    res = {}
    for name, e in (("plain", plain), ("coop", coop)):
        t, lg, ft = e.verify(toks.cuda(), pos)
        e.check()
        res[name] = (t.cpu(), lg.cpu(), ft.cpu())
    assert torch.equal(res["plain"][0], res["coop"][0])
    assert torch.equal(res["plain"][1], res["coop"][1])
    assert torch.equal(res["plain"][2], res["coop"][2])
    alt, ref = oracle_pair(orc, lambda: orc.forward(toks, pos)[0].float())
    check_rows(res["coop"][1], ref, alt, NAME, f"cooperative verify m={m}")


def test_cooperative_sampler_equals_plain(dev, monkeypatch):
    """fl_sample launched cooperatively and plainly: the same tokens and probabilities."""
    from flint_amd.generate import sample
    g = torch.Generator().manual_seed(3)
    lg = (torch.randn(16, 49152, generator=g) * 2).bfloat16().float().to(dev)
    t0, p0 = sample(lg, 0.8, 200, seed=9, offset=4, probs=True)
    torch.cuda.synchronize()
    monkeypatch.setenv("FLINT_AMD_COOPERATIVE", "1")
    t1, p1 = sample(lg, 0.8, 200, seed=9, offset=4, probs=True)
    torch.cuda.synchronize()
    assert torch.equal(t0, t1) and torch.equal(p0, p1)
    assert bool((t0 >= 0).all())
