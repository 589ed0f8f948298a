"""GPU parity of speculative verify (fl_verify: M tokens through all layers in one launch, the
GEMMs on the matrix cores) against the CPU oracle's masked forward.

Reference semantics (kernels/verify_mega.cu:106-283, spec_mega.py:51-57, spec_tree.py:46-51,
101-104): token m sits at cache slot pos+m, takes RoPE position pos+depth[m] and attends to the
cache [0, pos) plus the new tokens j with amask[m][j]. Known-answer structure of the reference's
own test (bench/verify_mega_test.py:43-59): a causal chain verified in one pass equals M
sequential decode steps. Tolerance as for decode: logits within logit_bar(config) (twice the
oracle's own fp32-order floor), argmax equal except where the oracle's top-2 margin is within it.
"""
import pytest
import torch

from tests.helpers import compare_logits, fill_kv_random, log, logit_bar, make_pair, near_tie

pytestmark = pytest.mark.gpu


def _check_rows(lg, lo, label, name):
    bar = logit_bar(name)
    ties = 0
    for m in range(lo.shape[0]):
        ok, d, within, same = compare_logits(lg[m], lo[m], name)
        am_e, am_o = int(torch.argmax(lg[m])), int(torch.argmax(lo[m]))
        log(f"{label} row {m}: max|dlogit|={d:.3e} ({within:.1%} within 2e-2) argmax {am_e}/{am_o}")
        assert ok, (label, m, d)
        if am_e != am_o:
            assert near_tie(lo[m], bar), (label, m)
            ties += 1
    return ties


@pytest.mark.parametrize("name,pos,m", [("tiny", 0, 5), ("tiny", 77, 8), ("small", 130, 5),
                                        ("small", 200, 16), ("tiny", 300, 1)])
def test_verify_chain_matches_oracle(dev, name, pos, m):
    args, sd, eng, orc = make_pair(name, seed=11)
    eng.setup_caches(1, 512)
    orc.setup_caches(eng.max_seq_length)
    fill_kv_random(eng, orc, pos, seed=pos + 3)
    g = torch.Generator().manual_seed(pos + m)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32)
    tout, lg, feat = eng.verify(toks.to(dev), pos)
    eng.check()
    lo, ho = orc.forward(toks, pos)
    ties = _check_rows(lg.cpu(), lo, f"{name} chain pos={pos} M={m}", name)
    assert ties <= 1
    assert torch.equal(tout.cpu(), torch.argmax(lg.cpu(), dim=-1).int())
    assert float((feat.cpu().float() - ho.float()).abs().max()) <= 0.25
    # the M new K / V rows were appended at slots pos .. pos+M-1
    for l in range(args.n_layer):
        kd = (eng.k_cache[l, :, pos:pos + m].float().cpu() - orc.k_cache[l, :, pos:pos + m].float()).abs()
        vd = (eng.v_cache[l, :, pos:pos + m].float().cpu() - orc.v_cache[l, :, pos:pos + m].float()).abs()
        assert float(torch.maximum(kd, vd).max()) <= 0.25, l


def test_verify_tree_matches_oracle(dev):
    """An 8-node draft tree (spec_tree.py:46-51): depth = node depth, amask = ancestors + self."""
    args, sd, eng, orc = make_pair("small", seed=12)
    eng.setup_caches(1, 512)
    orc.setup_caches(eng.max_seq_length)
    pos = 150
    fill_kv_random(eng, orc, pos, seed=21)
    parent = [-1, 0, 0, 1, 1, 2, 3, 5]
    m = len(parent)
    depth = torch.zeros(m, dtype=torch.int32)
    amask = torch.zeros(m, m, dtype=torch.uint8)
    for i in range(m):
        j = i
        while j >= 0:
            amask[i, j] = 1
            j = parent[j]
        depth[i] = int(amask[i].sum()) - 1
    toks = torch.randint(0, args.vocab_size, (m,), generator=torch.Generator().manual_seed(5),
                         dtype=torch.int32)
    tout, lg, feat = eng.verify(toks.to(dev), pos, depth=depth.to(dev), amask=amask.to(dev))
    eng.check()
    lo, ho = orc.forward(toks, pos, depth=depth, amask=amask)
    ties = _check_rows(lg.cpu(), lo, "tree", "small")
    assert ties <= 1


def test_verify_chain_equals_sequential_decode(dev):
    """Reference bench/verify_mega_test.py:43-59: verify of a causal chain == M decode steps."""
    args, sd, eng, _ = make_pair("tiny", seed=13)
    eng.setup_caches(1, 256)
    pos, m = 40, 6
    g = torch.Generator().manual_seed(9)
    prefix = torch.randint(0, args.vocab_size, (pos,), generator=g, dtype=torch.int32).to(dev)
    toks = torch.randint(0, args.vocab_size, (m,), generator=g, dtype=torch.int32).to(dev)
    from flint_amd.generate import prefill
    prefill(eng, prefix, 0)
    _, lg_v, _ = eng.verify(toks, pos)
    lg_v = lg_v.cpu()
    logits = torch.empty(args.vocab_size, dtype=torch.float32, device=dev)
    for i in range(m):
        eng.decode_step(toks[i:i + 1], pos + i, logits=logits)
        ok, d, within, same = compare_logits(logits.cpu(), lg_v[i], "tiny")
        log(f"chain step {i}: max|dlogit| verify vs decode {d:.3e} ({same:.1%} identical)")
        assert ok
    eng.check()


def test_verify_rejects_bad_arguments(dev):
    from flint_amd import _lib
    args, sd, eng, _ = make_pair("tiny", seed=1)
    eng.setup_caches(1, 64)
    toks = torch.zeros(17, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.FlError) as e:
        eng.verify(toks, 0)
    assert e.value.code == -3
    with pytest.raises(_lib.FlError) as e:
        eng.verify(toks[:4], 62)
    assert e.value.code == -2
